/*
 * mi_attn.h — C ABI of the MI355X (gfx950) attention library for the
 * Qwen3.6 full-attention layers: GQA decode over an f16 KV cache, causal
 * batched prefill, K-token speculative verify, ragged batched decode, and the
 * KV-cache append / reset / rollback state those steps read and write.
 *
 * Conventions
 *   - Every entry point returns an mi_status; nothing aborts across the ABI.
 *     On failure mi_last_error() returns a thread-local description.
 *   - Tensor arguments are DEVICE pointers unless the parameter name starts
 *     with "host_".  f16 values are IEEE binary16 bit patterns (mi_f16).
 *   - Work is enqueued on the caller's stream (a hipStream_t passed as void*;
 *     NULL is the legacy default stream) and is asynchronous unless the name
 *     ends in _sync.  A handle is not internally synchronised: use one handle
 *     per thread (the reference's pyclasses are `unsendable`).  The decode,
 *     step and verify calls of one handle share its split-K workspace, so
 *     issue them on one stream (or order the streams with events): two of
 *     them running concurrently on different streams race on it.
 *   - Graph capture: the calls allocate and clear nothing once the cache and
 *     the handle's workspace are large enough, so they can be captured.  A
 *     call that would have to grow either while its stream is capturing
 *     returns MI_ERR_INVALID_ARG; make one eager call of the largest size
 *     (or mi_kv_reserve) first.  A workspace replaced by a larger one after
 *     a capture used it is kept until mi_kv_destroy, so graphs captured
 *     earlier stay valid (one never captured is freed when replaced); cache
 *     growth (mi_kv_reserve, or an append past capacity) moves the K/V
 *     buffers and invalidates every graph captured on the handle.
 *   - A handle belongs to the device that is current at mi_kv_create; calls
 *     that allocate or launch work on it return MI_ERR_INVALID_ARG unless
 *     that device is current.
 *   - Shapes: H query heads, G KV heads, head dim D.  The kernels are built
 *     for the Qwen3.6 full-attention shape D = 256, H / G = 8; other shapes
 *     return MI_ERR_UNSUPPORTED.  Softmax scale is 1/sqrt(D), accumulation f32.
 *
 * Logical KV layout is the reference's token-major K[pos][kvh*D + i]
 * (src/math_util.rs:336); mi_kv_upload / mi_kv_download convert to and from
 * token-major host rows, so callers that move cache contents through the
 * host see the reference layout.  Physical layout on the device (what
 * mi_kv_layer_ptrs, mi_kv_pack and mi_attn_decode_ragged see), chosen so
 * that the MFMA operands of the decode kernel are whole 16-byte vectors and
 * each 16-lane group of a wave reads 256 contiguous bytes:
 *   K: 32-row blocks.  Row r = 32*b + w, element (r, h, i) at
 *        K + (((b*G + h)*2 + u)*(D/8) + i/8)*128 + j*8 + i%8,
 *      u = (w/4) % 2, j = 4*(w/8) + w%4.
 *   V: 8-row transposed blocks: element (r, h, i) at
 *        V + ((r/8)*G + h)*D*8 + i*8 + r%8
 *      so the eight keys of one value column are one 16-byte load.
 */
#ifndef MI_ATTN_H
#define MI_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t mi_f16;
typedef void* mi_stream;

typedef enum mi_status {
  MI_OK = 0,
  MI_ERR_INVALID_ARG = 1,   /* null pointer, bad layer, n <= 0, bad shape   */
  MI_ERR_OUT_OF_RANGE = 2,  /* position beyond capacity / sequence length   */
  MI_ERR_OOM = 3,           /* device allocation failed                     */
  MI_ERR_HIP = 4,           /* a HIP runtime call failed                    */
  MI_ERR_UNSUPPORTED = 5    /* head shape the kernels are not built for     */
} mi_status;

/* Rows per K block and per V block of the device layout, and the
 * granularity capacities are rounded up to. */
#define MI_KV_KBLOCK 32
#define MI_KV_VBLOCK 8
#define MI_KV_CAP_ALIGN 256

/* Roofline constants every measurement in this project divides by
 * (MI355X datasheet: HBM3E 8.0 TB/s, dense f16 MFMA 2.5 PFLOP/s). */
#define MI_PEAK_HBM_GBPS 8000.0
#define MI_PEAK_F16_TFLOPS 2500.0

/* ---------------------------------------------------------------- errors -- */

/* Thread-local message of the last failed call on this thread ("" if none).
 * Replaces MoEError's Display (src/error.rs:4-9). */
const char* mi_last_error(void);

/* Version / build string, e.g. "mi_attn 0.1 gfx950". */
const char* mi_version(void);

/* Writes MI_PEAK_HBM_GBPS and MI_PEAK_F16_TFLOPS (for bindings that cannot
 * read macros). */
void mi_roofline_peaks(double* hbm_gbps, double* f16_tflops);

/* -------------------------------------------------------------- KV cache -- */

typedef struct mi_kv mi_kv;

/* Per-full-attention-layer K/V store plus `pos` and per-layer `len`.
 * Replaces Cache::new (src/cache.rs:45-76) and the GPU buffers of
 * MetalContext (src/engine/qwen35_moe/metal_context.rs:316-319, 492-502).
 * `num_layers` counts full-attention layers only (the reference's Linear
 * layers hold no KV).  Capacity is rounded up to MI_KV_CAP_ALIGN rows; new
 * memory is zero-filled.  Blocks until allocation and clearing finish. */
mi_status mi_kv_create(int32_t num_layers, int32_t num_q_heads,
                       int32_t num_kv_heads, int32_t head_dim,
                       int64_t capacity, mi_kv** out);
void mi_kv_destroy(mi_kv* kv);

/* Grow to at least `capacity` rows, keeping every existing row (including
 * stale rows past len, as metal_context.rs:368-431 copies the whole old
 * buffer).  Never shrinks.  Synchronous. */
mi_status mi_kv_reserve(mi_kv* kv, int64_t capacity);
mi_status mi_kv_capacity(const mi_kv* kv, int64_t* capacity);
mi_status mi_kv_shape(const mi_kv* kv, int32_t* num_layers, int32_t* num_q_heads,
                      int32_t* num_kv_heads, int32_t* head_dim);

/* Cache::set_pos (src/cache.rs:102-109): pos = p and len = p on every layer.
 * Rollback is position-only: no row is modified. */
mi_status mi_kv_set_pos(mi_kv* kv, int64_t pos);
/* Cache::reset (src/cache.rs:84-94) restricted to KV state: set_pos(0). */
mi_status mi_kv_reset(mi_kv* kv);
mi_status mi_kv_pos(const mi_kv* kv, int64_t* pos);
mi_status mi_kv_len(const mi_kv* kv, int32_t layer, int64_t* len);
/* FullState::len of one layer (src/cache.rs:273-287); p <= capacity. */
mi_status mi_kv_set_len(mi_kv* kv, int32_t layer, int64_t len);

/* Device base pointers of one layer (physical layout above). */
mi_status mi_kv_layer_ptrs(mi_kv* kv, int32_t layer, mi_f16** k, mi_f16** v);

/* kv_cache_append / kv_cache_append_n (src/math_util.rs:387-392,
 * src/engine/shaders.metal:2370-2383, 2774-2792): bit copy of n rows of
 * G*D values from k[n][G*D], v[n][G*D] into rows [pos, pos+n); then
 * len(layer) = pos + n (src/engine/qwen35_moe/cpu.rs:144).  Grows the cache
 * (synchronously) when pos + n exceeds capacity. */
mi_status mi_kv_append(mi_kv* kv, int32_t layer, const mi_f16* k,
                       const mi_f16* v, int64_t pos, int32_t n,
                       mi_stream stream);

/* Host <-> device copies of rows [row0, row0+rows) of one layer in
 * token-major order (MetalContext::upload_cache / download_cache,
 * metal_context.rs:804-882).  Synchronous.  Upload does not change len. */
mi_status mi_kv_upload(mi_kv* kv, int32_t layer, const mi_f16* host_k,
                       const mi_f16* host_v, int64_t row0, int64_t rows);
mi_status mi_kv_download(const mi_kv* kv, int32_t layer, mi_f16* host_k,
                         mi_f16* host_v, int64_t row0, int64_t rows);

/* Cache::copy_from (src/cache.rs:112-128): copies every row of every layer,
 * pos and len.  Shapes must match; dst grows to src's capacity.  Synchronous. */
mi_status mi_kv_copy_from(mi_kv* dst, const mi_kv* src);

/* ------------------------------------------------------------- attention -- */

/* Decode attention of one query token over rows [0, seq_len) of `layer`:
 * out[h] = softmax(q_h . K^T / sqrt(D)) V  for every query head h, KV head
 * h / (H/G); then out *= sigmoid(gate) elementwise when gate != NULL.
 * q, gate, out: [H*D] f16.  Split-K flash-decoding plus a combine kernel.
 * Semantics: attention_scores/softmax/values_batched + sigmoid_gate_inplace
 * (src/math_util.rs:264-269, 323-383), kernels attn_sdpa_block +
 * attn_sdpa_reduce (src/engine/shaders.metal:1559-1776).  seq_len == 0 gives
 * zeros (the reference's zero-filled output, math_util.rs:372). */
mi_status mi_attn_decode(mi_kv* kv, int32_t layer, const mi_f16* q,
                         const mi_f16* gate, mi_f16* out, int64_t seq_len,
                         mi_stream stream);

/* The engine's full-attention step for one token (encode_pre_expert_full,
 * src/engine/qwen35_moe/fused_exp2.rs:669-733; cpu.rs:136-167): append k, v
 * ([G*D] f16) at `pos`, then decode with seq_len = pos + 1 and gate.
 * Leaves pos(kv) unchanged: the engine advances it once per token, after
 * its last layer, with mi_kv_set_pos(pos + 1) (fused_exp2.rs:1030-1031). */
mi_status mi_attn_step(mi_kv* kv, int32_t layer, const mi_f16* q,
                       const mi_f16* k, const mi_f16* v, const mi_f16* gate,
                       mi_f16* out, int64_t pos, mi_stream stream);

/* Causal batched prefill (op1_full_batched, src/engine/qwen35_moe/
 * batched.rs:233-260; kernels kv_cache_append_n + attn_sdpa_causal_n,
 * shaders.metal:2656-2792): append n rows k, v [n][G*D] at past_pos, then
 * query i (q [n][H][D]) attends rows [0, past_pos + i] inclusive; gate
 * [n][H][D] or NULL; out [n][H][D].  MFMA flash-attention kernel; up to
 * 1024 new tokens after a past of at least 2048 rows (and twice n) run its
 * split-K form over key chunks plus a merge, which needs the handle's
 * workspace (grown on demand; under graph capture only when it already
 * suffices, else the unsplit kernel runs).  MI_ATTN_PREFILL_SPLIT=0 turns
 * the split-K form off.
 * k = v = NULL: rows [past_pos, past_pos+n) are already in the cache (written
 * by mi_qk_norm_rope_append or mi_kv_append; len(layer) >= past_pos + n), no
 * append; len(layer) becomes past_pos + n. */
mi_status mi_attn_prefill(mi_kv* kv, int32_t layer, const mi_f16* q,
                          const mi_f16* k, const mi_f16* v, const mi_f16* gate,
                          mi_f16* out, int64_t past_pos, int32_t n,
                          mi_stream stream);

/* K-token verify for speculative decoding: same contract as mi_attn_prefill
 * (append at past_pos, query i attends [0, past_pos + i]) for small n, run
 * split-K over the cache: up to 4 tokens in the decode kernel's form, more
 * in one pass of the prefill's MFMA tiles over key chunks that reads each
 * K/V tile once per 16 tokens (MI_ATTN_VERIFY_WIDE=0 runs them as 4-token
 * groups instead), then a merge.  Rollback afterwards is
 * mi_kv_set_pos.  k = v = NULL as for mi_attn_prefill. */
mi_status mi_attn_verify(mi_kv* kv, int32_t layer, const mi_f16* q,
                         const mi_f16* k, const mi_f16* v, const mi_f16* gate,
                         mi_f16* out, int64_t past_pos, int32_t n,
                         mi_stream stream);

/* Ragged batched decode: `batch` independent sequences, one query token
 * each.  Sequence s owns rows [offsets[s], offsets[s] + lengths[s]) of the
 * shared k_rows / v_rows buffers (physical layout above with G KV heads;
 * offsets must be multiples of MI_KV_KBLOCK, the buffers must hold whole
 * blocks).  offsets, lengths: device int32[batch].  q, gate, out:
 * [batch][H][D].  max_len >= every lengths[s]; batch <= 65535 (else
 * MI_ERR_UNSUPPORTED).  The sequences' 32-row tiles are split evenly over the
 * CUs (one launch attends, one merges; the attending launch computes the
 * tile offsets itself for up to 256 sequences, a launch before it does for
 * larger batches), so a batch of unequal lengths keeps every CU busy.
 * No reference counterpart (the reference decodes one sequence,
 * README.md:150-165); per-sequence math is mi_attn_decode's.  Needs a
 * device workspace of mi_attn_ragged_workspace_size bytes. */
size_t mi_attn_ragged_workspace_size(int32_t batch, int32_t max_len,
                                     int32_t num_q_heads, int32_t num_kv_heads,
                                     int32_t head_dim);
mi_status mi_attn_decode_ragged(const mi_f16* k_rows, const mi_f16* v_rows,
                                const int32_t* offsets, const int32_t* lengths,
                                int32_t batch, int32_t max_len,
                                int32_t num_q_heads, int32_t num_kv_heads,
                                int32_t head_dim, const mi_f16* q,
                                const mi_f16* gate, mi_f16* out,
                                void* workspace, size_t workspace_bytes,
                                mi_stream stream);

/* Bytes of the device-resident scratch array behind
 * mi_attn_decode_ragged_noalloc (one copy per device, held until the process
 * ends): 16 MiB, which covers batches up to 887 sequences at the Qwen3.6
 * shape (16 query / 2 KV heads, head_dim 256) with the default split (one KV
 * head per workgroup); MI_ATTN_SPLIT_GH=2 lowers that to 759.  The exact
 * test is mi_attn_ragged_workspace_size(...) <= MI_NOALLOC_SCRATCH_BYTES. */
#define MI_NOALLOC_SCRATCH_BYTES (16u << 20)

/* mi_attn_decode_ragged without a workspace argument, for callers that
 * cannot allocate device memory (code under graph capture, serving loops
 * and harnesses that forbid hipMalloc): the workspace is a file-scope
 * device array of MI_NOALLOC_SCRATCH_BYTES.  The call allocates and frees
 * nothing; a batch whose mi_attn_ragged_workspace_size exceeds the array
 * returns MI_ERR_UNSUPPORTED.  Every call on one device shares that
 * device's array: calls that overlap in time on one device (other streams
 * or threads) race on it and must be serialised by the caller.  The stream
 * must belong to the current device (MI_ERR_INVALID_ARG otherwise).  Same
 * arguments and results as mi_attn_decode_ragged otherwise.
 * No counterpart in the reference (whose decode is single-sequence). */
mi_status mi_attn_decode_ragged_noalloc(const mi_f16* k_rows, const mi_f16* v_rows,
                                        const int32_t* offsets, const int32_t* lengths,
                                        int32_t batch, int32_t max_len,
                                        int32_t num_q_heads, int32_t num_kv_heads,
                                        int32_t head_dim, const mi_f16* q,
                                        const mi_f16* gate, mi_f16* out,
                                        mi_stream stream);

/* Layout helper for callers that build ragged buffers themselves: writes
 * `rows` token-major rows k_rows, v_rows ([rows][G*D]) at rows
 * [row0, row0+rows) of dst_k / dst_v in the device layout above (rows of
 * partially covered blocks outside the range are kept).  Async. */
mi_status mi_kv_pack(const mi_f16* k_rows, const mi_f16* v_rows, mi_f16* dst_k,
                     mi_f16* dst_v, int64_t row0, int64_t rows,
                     int32_t num_kv_heads, int32_t head_dim, mi_stream stream);

/* ----------------------------------------------- Q/K head norm + RoPE -- */

/* Largest rotary_dim mi_qk_norm_rope_append accepts. */
#define MI_ROPE_MAX_DIM 256

/* The step before attention, fused: per-head RMS norm of Q and K with bf16
 * weights, NeoX partial rotary embedding of the first rotary_dim columns at
 * position pos + t for token t, the Q/gate split of q_proj, and the append of
 * the rotated K and the raw V rows at rows [pos, pos+n) of `layer`; then
 * len(layer) = pos + n (grows the cache synchronously like mi_kv_append).
 * Replaces q_head_norm_rope + k_head_norm_rope + kv_cache_append
 * (src/math_util.rs:387-392, 501-593; src/engine/shaders.metal:2244-2383;
 * called at src/engine/qwen35_moe/cpu.rs:126-145, fused_exp2.rs:630-680).
 * q_proj: [n][H][2*D] f32, each head's query then gate; k, v: [n][G][D] f32;
 * q_norm_w, k_norm_w: bf16 bit patterns [D]; q_out, gate_out: [n][H][D] f16.
 * rotary_dim: multiple of 8, at most min(D, MI_ROPE_MAX_DIM) (the reference
 * uses 64 = partial_rotary_factor * head_dim, rope_theta 1e7, eps 1e-6,
 * qwen35_moe/constants.rs:166-167).  Async on `stream`. */
mi_status mi_qk_norm_rope_append(mi_kv* kv, int32_t layer, const float* q_proj,
                                 const float* k, const float* v,
                                 const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                 int32_t rotary_dim, float rope_theta, float eps,
                                 int64_t pos, int32_t n, mi_f16* q_out,
                                 mi_f16* gate_out, mi_stream stream);

/* The whole full-attention step of one token from its projections, in the
 * two kernels of mi_attn_step: Q and K per-head RMS norm + NeoX RoPE at
 * position pos (as mi_qk_norm_rope_append), append of the rotated K and raw V
 * at row pos, decode with seq_len = pos + 1 and the sigmoid gate taken from
 * the gate halves of q_proj.  Replaces q_head_norm_rope, k_head_norm_rope,
 * kv_cache_append, attn_sdpa_block, attn_sdpa_reduce and sigmoid_gate of
 * encode_pre_expert_full (src/engine/qwen35_moe/fused_exp2.rs:630-733;
 * CPU form cpu.rs:126-167).  q_proj: [H][2*D] f32; k, v: [G][D] f32;
 * weights bf16 [D]; out: [H*D] f16.  rotary_dim must be a multiple of 64
 * (else MI_ERR_UNSUPPORTED: use mi_qk_norm_rope_append + mi_attn_decode).
 * len(layer) = pos + 1; pos(kv) is unchanged, as for mi_attn_step. */
mi_status mi_attn_step_proj(mi_kv* kv, int32_t layer, const float* q_proj,
                            const float* k, const float* v,
                            const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                            int32_t rotary_dim, float rope_theta, float eps,
                            mi_f16* out, int64_t pos, mi_stream stream);

/* ------------------------------------------------------------- o_proj -- */

/* o_proj of the gated attention output: out[r] = sum_c W[r][c] * x[c] for
 * r < out_dim, W [out_dim][in_dim] bf16 (bit patterns), x [in_dim] f16 (the
 * output of mi_attn_decode / mi_attn_step with the gate), out f32.  Replaces
 * the BF16 matvec of the o_proj (matvec_bf16, src/engine/shaders.metal:
 * 2392-2425; dispatched at src/engine/qwen35_moe/fused_exp2.rs:732).
 * in_dim must be a multiple of 512.  Async. */
mi_status mi_matvec_bf16(const mi_f16* x, const uint16_t* w, float* out,
                         int32_t out_dim, int32_t in_dim, mi_stream stream);

/* The same with the reference's 4-bit affine weights (dequant_matvec_4bit,
 * src/math_util.rs:14-57): w_packed [out_dim][in_dim/8] u32, eight nibbles
 * per word, low nibble first = the lower column; scales, biases bf16
 * [out_dim][in_dim/group_size]; weight = nibble * scale + bias.  in_dim a
 * multiple of 2048, group_size a multiple of 32 dividing in_dim.  Async. */
mi_status mi_matvec_q4(const mi_f16* x, const uint32_t* w_packed,
                       const uint16_t* scales, const uint16_t* biases,
                       int32_t group_size, float* out, int32_t out_dim,
                       int32_t in_dim, mi_stream stream);

/* ------------------------------------------------------------- profiling -- */

/* Kernel timing with HIP events stamped by each dispatch on its launch
 * stream (the reference's telemetry counterpart, src/engine.rs:13-24, at
 * kernel granularity).  mi_prof_enable synchronises the device and clears
 * earlier records.  Kernel names: "attn_split", "attn_combine",
 * "attn_prefill", "kv_pack",
 * "qk_norm_rope", "matvec_bf16", "matvec_q4", "ragged_plan".
 * mi_prof_read returns the mean duration in microseconds and the number of
 * launches recorded since the last enable. */
void mi_prof_enable(int on);
mi_status mi_prof_read(const char* kernel, double* avg_us, int64_t* count);

/* MFMA issue ceiling (measurement only; no counterpart in the reference):
 * `workgroups` workgroups of 4 waves, one wave per SIMD, each issuing
 * `iters` x 8 v_mfma_f32_32x32x16_f16 back to back (4 independent chains,
 * A rotating over 8 register fragments, no LDS / VALU / memory in the loop).
 * `operands` holds (8 + 4) x 8 halves per thread of a workgroup (256
 * threads, 24 KiB; all workgroups read the same ones); `out` receives one
 * float per thread (workgroups x 256) so nothing is optimised away;
 * `clocks` receives per workgroup the shader-clock cycles and the 100 MHz
 * reference-clock ticks of its loop.  bench.py prices the prefill against
 * what this reaches with random and with zero operands.  Kernel name for
 * mi_prof_read: "mfma_ceiling". */
mi_status mi_bench_mfma_ceiling(const mi_f16* operands, int32_t iters, int32_t workgroups,
                                float* out, uint64_t* clocks, mi_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_ATTN_H */
