/*
 * attn_oracle.c — CPU restatement of the reference's full-attention math.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernels are
 * compared against (tests/, __graft_entry__.smoke, and the cpu_baseline leg
 * of bench.py).  The product library never links, loads or calls it.
 *
 * Reference: fbundle/moe_infer (Rust).  Each function names the file:line it
 * restates.  The reference KV cache is f32 (src/cache.rs:280-286); the build
 * stores f16, so the *_f16 entry points widen f16 inputs to f32 exactly and
 * then run the reference's f32 loops unchanged.  The *_f64 twins run the
 * same loop order in double precision and serve as the high-precision
 * expected value for tolerance tests.
 *
 * Pinning (no golden vectors exist in the reference for this path): the
 * tests in tests/test_oracle.py check every function here against an
 * independent numpy/scipy evaluation (einsum + scipy.special.softmax in
 * f64), against closed forms (seq_len 1, equal keys, q = 0, dominant key,
 * sigmoid(0) = 1/2, permutation invariance, causal row i == decode at
 * past+i+1) and the f16 conversions exhaustively against numpy.float16.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifndef ORACLE_CFLAGS
#define ORACLE_CFLAGS "unknown"
#endif
/* The compiler and flags this library was built with (reported beside the
   CPU baseline timings). */
const char* oracle_build_info(void) { return "gcc " __VERSION__ ", " ORACLE_CFLAGS; }

#define ORACLE_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ f16 -- */

/* IEEE binary16 -> binary32, exact (every half is a float). */
ORACLE_API float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do { man <<= 1; e++; } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* binary32 -> binary16, round to nearest even (IEEE default). */
ORACLE_API uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) { /* inf or nan */
    if (absx > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((absx >> 13) & 0x3ffu));
    return (uint16_t)(sign | 0x7c00u);
  }
  if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  int32_t e = (int32_t)(absx >> 23) - 127;
  if (e >= -14) { /* normal half */
    uint32_t man = absx & 0x7fffffu;
    uint32_t half = ((uint32_t)(e + 15) << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
    return (uint16_t)(sign | half);
  }
  if (e < -25) return (uint16_t)sign; /* below half of the smallest subnormal */
  { /* subnormal half: value = m * 2^-24 */
    uint32_t man = (absx & 0x7fffffu) | 0x800000u; /* 24-bit significand */
    int shift = -e - 14 + 13;                      /* 14 .. 24 */
    uint32_t half = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1u))) half++;
    return (uint16_t)(sign | half);
  }
}

ORACLE_API void oracle_widen_f16(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = oracle_f16_to_f32(src[i]);
}

ORACLE_API void oracle_narrow_f32(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; i++) dst[i] = oracle_f32_to_f16(src[i]);
}

/* --------------------------------------------- reference f32 functions -- */

/* src/math_util.rs:323-342  attention_scores_batched */
ORACLE_API void oracle_attention_scores_batched(
    const float* q, const float* k_cache, float* scores, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t kv_dim, int64_t seq_len,
    int64_t max_seq) {
  float scale = 1.0f / sqrtf((float)head_dim);
  int64_t n_rep = num_q_heads / num_kv_heads;
  for (int64_t qh = 0; qh < num_q_heads; qh++) {
    int64_t kh = qh / n_rep;
    const float* q_head = q + qh * head_dim;
    int64_t k_head_base = kh * head_dim;
    float* scores_row = scores + qh * max_seq;
    for (int64_t t = 0; t < seq_len; t++) {
      const float* k_t = k_cache + t * kv_dim + k_head_base;
      float dot = 0.0f;
      for (int64_t d = 0; d < head_dim; d++) dot += q_head[d] * k_t[d];
      scores_row[t] = dot * scale;
    }
  }
}

/* src/math_util.rs:346-360  attention_softmax_batched */
ORACLE_API void oracle_attention_softmax_batched(float* scores,
                                                 int64_t num_q_heads,
                                                 int64_t seq_len,
                                                 int64_t max_seq) {
  for (int64_t h = 0; h < num_q_heads; h++) {
    float* s = scores + h * max_seq;
    float max_val = -INFINITY;
    for (int64_t t = 0; t < seq_len; t++) max_val = fmaxf(max_val, s[t]);
    float sum = 0.0f;
    for (int64_t t = 0; t < seq_len; t++) {
      s[t] = expf(s[t] - max_val);
      sum += s[t];
    }
    if (sum > 0.0f) {
      float inv = 1.0f / sum;
      for (int64_t t = 0; t < seq_len; t++) s[t] *= inv;
    }
  }
}

/* src/math_util.rs:365-383  attention_values_batched */
ORACLE_API void oracle_attention_values_batched(
    const float* scores, const float* v_cache, float* out, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t kv_dim, int64_t seq_len,
    int64_t max_seq) {
  int64_t n_rep = num_q_heads / num_kv_heads;
  memset(out, 0, sizeof(float) * (size_t)(num_q_heads * head_dim));
  for (int64_t qh = 0; qh < num_q_heads; qh++) {
    int64_t kh = qh / n_rep;
    const float* scores_row = scores + qh * max_seq;
    int64_t v_head_base = kh * head_dim;
    float* out_row = out + qh * head_dim;
    for (int64_t t = 0; t < seq_len; t++) {
      float s = scores_row[t];
      const float* v_t = v_cache + t * kv_dim + v_head_base;
      for (int64_t d = 0; d < head_dim; d++) out_row[d] += s * v_t[d];
    }
  }
}

/* src/math_util.rs:387-392  kv_cache_append */
ORACLE_API void oracle_kv_cache_append(const float* k, const float* v,
                                       float* k_cache, float* v_cache,
                                       int64_t pos, int64_t kv_dim) {
  memcpy(k_cache + pos * kv_dim, k, sizeof(float) * (size_t)kv_dim);
  memcpy(v_cache + pos * kv_dim, v, sizeof(float) * (size_t)kv_dim);
}

/* src/math_util.rs:264-269  sigmoid_gate_inplace */
ORACLE_API void oracle_sigmoid_gate_inplace(float* out, const float* gate,
                                            int64_t dim) {
  for (int64_t i = 0; i < dim; i++) {
    float g = 1.0f / (1.0f + expf(-gate[i]));
    out[i] *= g;
  }
}

/* One decode step of the reference's f32 attention core (the four functions
 * above, in the order cpu.rs:149-163 calls them), with the query heads
 * spread over `threads` OpenMP threads.  Each head runs the same scalar
 * loops as the batched functions (called with one head and the head's K / V
 * column offset), so the result equals the single-threaded one bit for bit.
 * A CPU baseline variant only; the reference runs its attention on one
 * thread. */
ORACLE_API void oracle_decode_heads_omp(const float* q, const float* k_cache,
                                        const float* v_cache, const float* gate,
                                        float* scores, float* out, int64_t num_q_heads,
                                        int64_t num_kv_heads, int64_t head_dim,
                                        int64_t kv_dim, int64_t seq_len, int64_t max_seq,
                                        int threads) {
  const int64_t n_rep = num_q_heads / num_kv_heads;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t qh = 0; qh < num_q_heads; qh++) {
    const int64_t kh = qh / n_rep;
    float* s = scores + qh * max_seq;
    oracle_attention_scores_batched(q + qh * head_dim, k_cache + kh * head_dim, s, 1, 1,
                                    head_dim, kv_dim, seq_len, max_seq);
    oracle_attention_softmax_batched(s, 1, seq_len, max_seq);
    oracle_attention_values_batched(s, v_cache + kh * head_dim, out + qh * head_dim, 1, 1,
                                    head_dim, kv_dim, seq_len, max_seq);
    if (gate) oracle_sigmoid_gate_inplace(out + qh * head_dim, gate + qh * head_dim, head_dim);
  }
}

/* src/engine/qwen35_moe/mtp.rs:304-350  cpu_attention (MTP layer form:
 * normalisation by sum_exp inside the P.V loop, no sum > 0 guard). */
ORACLE_API void oracle_mtp_cpu_attention(const float* q, const float* k_cache,
                                         const float* v_cache, float* out,
                                         int64_t num_heads,
                                         int64_t num_kv_heads,
                                         int64_t head_dim, int64_t seq_len,
                                         float kq_scale) {
  int64_t kv_dim = num_kv_heads * head_dim;
  int64_t group_size = num_heads / num_kv_heads;
  float* scores = (float*)malloc(sizeof(float) * (size_t)(seq_len > 0 ? seq_len : 1));
  for (int64_t h = 0; h < num_heads; h++) {
    int64_t kv_h = h / group_size;
    int64_t q_off = h * head_dim;
    float max_score = -INFINITY;
    for (int64_t t = 0; t < seq_len; t++) {
      int64_t k_off = t * kv_dim + kv_h * head_dim;
      float dot = 0.0f;
      for (int64_t d = 0; d < head_dim; d++) dot += q[q_off + d] * k_cache[k_off + d];
      scores[t] = dot * kq_scale;
      max_score = fmaxf(max_score, scores[t]);
    }
    float sum_exp = 0.0f;
    for (int64_t t = 0; t < seq_len; t++) {
      scores[t] = expf(scores[t] - max_score);
      sum_exp += scores[t];
    }
    for (int64_t d = 0; d < head_dim; d++) {
      float acc = 0.0f;
      for (int64_t t = 0; t < seq_len; t++) {
        int64_t v_off = t * kv_dim + kv_h * head_dim;
        acc += scores[t] / sum_exp * v_cache[v_off + d];
      }
      out[q_off + d] = acc;
    }
  }
  free(scores);
}

/* ------------------------------------------------ composed attention step -- */

/* One decode step's attention core, in the order of
 * src/engine/qwen35_moe/cpu.rs:146-167: scores -> softmax -> values ->
 * sigmoid gate (gate may be NULL: no gating).  K/V rows are token-major
 * f32 [seq_len][G*D] (the cache contents after the append at cpu.rs:141).
 * `scores` is scratch of num_q_heads*seq_len floats (max_seq = seq_len). */
ORACLE_API void oracle_attn_decode_f32(const float* q, const float* gate,
                                       const float* k_rows,
                                       const float* v_rows, int64_t H,
                                       int64_t G, int64_t D, int64_t seq_len,
                                       float* out) {
  int64_t ms = seq_len > 0 ? seq_len : 1;
  float* scores = (float*)calloc((size_t)(H * ms), sizeof(float));
  oracle_attention_scores_batched(q, k_rows, scores, H, G, D, G * D, seq_len, ms);
  oracle_attention_softmax_batched(scores, H, seq_len, ms);
  oracle_attention_values_batched(scores, v_rows, out, H, G, D, G * D, seq_len, ms);
  if (gate) oracle_sigmoid_gate_inplace(out, gate, H * D);
  free(scores);
}

/* Same on f16 bit patterns: widen q, gate, K, V exactly to f32 and run the
 * reference f32 loops. */
ORACLE_API void oracle_attn_decode_f16(const uint16_t* q, const uint16_t* gate,
                                       const uint16_t* k_rows,
                                       const uint16_t* v_rows, int64_t H,
                                       int64_t G, int64_t D, int64_t seq_len,
                                       float* out) {
  int64_t nkv = seq_len * G * D;
  float* qf = (float*)malloc(sizeof(float) * (size_t)(H * D));
  float* gf = gate ? (float*)malloc(sizeof(float) * (size_t)(H * D)) : NULL;
  float* kf = (float*)malloc(sizeof(float) * (size_t)(nkv > 0 ? nkv : 1));
  float* vf = (float*)malloc(sizeof(float) * (size_t)(nkv > 0 ? nkv : 1));
  oracle_widen_f16(q, qf, H * D);
  if (gate) oracle_widen_f16(gate, gf, H * D);
  oracle_widen_f16(k_rows, kf, nkv);
  oracle_widen_f16(v_rows, vf, nkv);
  oracle_attn_decode_f32(qf, gf, kf, vf, H, G, D, seq_len, out);
  free(qf); free(gf); free(kf); free(vf);
}

/* Causal batched attention, src/engine/shaders.metal:2656-2769
 * (attn_sdpa_causal_n): query i (position past_pos + i) attends rows
 * [0, past_pos + i] inclusive.  Its arithmetic is the decode step above at
 * seq_len = past_pos + i + 1, which is how the reference's CPU engine would
 * run the same tokens one at a time (cpu.rs:141-167).  q, gate, out:
 * [n][H][D]; K/V rows token-major [past_pos + n][G*D] (after the append of
 * batched.rs:233-238). */
ORACLE_API void oracle_attn_causal_n_f16(const uint16_t* q,
                                         const uint16_t* gate,
                                         const uint16_t* k_rows,
                                         const uint16_t* v_rows, int64_t H,
                                         int64_t G, int64_t D,
                                         int64_t past_pos, int64_t n,
                                         float* out) {
  int64_t rows = past_pos + n;
  int64_t nkv = rows * G * D;
  float* kf = (float*)malloc(sizeof(float) * (size_t)(nkv > 0 ? nkv : 1));
  float* vf = (float*)malloc(sizeof(float) * (size_t)(nkv > 0 ? nkv : 1));
  float* qf = (float*)malloc(sizeof(float) * (size_t)(H * D));
  float* gf = (float*)malloc(sizeof(float) * (size_t)(H * D));
  oracle_widen_f16(k_rows, kf, nkv);
  oracle_widen_f16(v_rows, vf, nkv);
  for (int64_t i = 0; i < n; i++) {
    oracle_widen_f16(q + i * H * D, qf, H * D);
    if (gate) oracle_widen_f16(gate + i * H * D, gf, H * D);
    oracle_attn_decode_f32(qf, gate ? gf : NULL, kf, vf, H, G, D, past_pos + i + 1,
                           out + i * H * D);
  }
  free(kf); free(vf); free(qf); free(gf);
}

/* Ragged batch of independent decode steps: sequence s uses token-major rows
 * [offsets[s], offsets[s] + lengths[s]) of k_rows / v_rows. */
ORACLE_API void oracle_attn_decode_ragged_f16(
    const uint16_t* q, const uint16_t* gate, const uint16_t* k_rows,
    const uint16_t* v_rows, const int32_t* offsets, const int32_t* lengths,
    int64_t batch, int64_t H, int64_t G, int64_t D, float* out) {
  for (int64_t s = 0; s < batch; s++) {
    int64_t off = (int64_t)offsets[s] * G * D;
    oracle_attn_decode_f16(q + s * H * D, gate ? gate + s * H * D : NULL,
                           k_rows + off, v_rows + off, H, G, D, lengths[s],
                           out + s * H * D);
  }
}

/* ------------------------------------------------------------ f64 twins -- */

/* The decode step of oracle_attn_decode_f32 in double precision, same loop
 * order, inputs f16 widened exactly. */
ORACLE_API void oracle_attn_decode_f64(const uint16_t* q, const uint16_t* gate,
                                       const uint16_t* k_rows,
                                       const uint16_t* v_rows, int64_t H,
                                       int64_t G, int64_t D, int64_t seq_len,
                                       double* out) {
  double scale = 1.0 / sqrt((double)D);
  int64_t n_rep = H / G, kv_dim = G * D;
  double* s = (double*)malloc(sizeof(double) * (size_t)(seq_len > 0 ? seq_len : 1));
  for (int64_t qh = 0; qh < H; qh++) {
    int64_t kh = qh / n_rep;
    double mx = -INFINITY;
    for (int64_t t = 0; t < seq_len; t++) {
      double dot = 0.0;
      for (int64_t d = 0; d < D; d++)
        dot += (double)oracle_f16_to_f32(q[qh * D + d]) *
               (double)oracle_f16_to_f32(k_rows[t * kv_dim + kh * D + d]);
      s[t] = dot * scale;
      if (s[t] > mx) mx = s[t];
    }
    double sum = 0.0;
    for (int64_t t = 0; t < seq_len; t++) { s[t] = exp(s[t] - mx); sum += s[t]; }
    if (sum > 0.0) for (int64_t t = 0; t < seq_len; t++) s[t] /= sum;
    for (int64_t d = 0; d < D; d++) {
      double acc = 0.0;
      for (int64_t t = 0; t < seq_len; t++)
        acc += s[t] * (double)oracle_f16_to_f32(v_rows[t * kv_dim + kh * D + d]);
      if (gate) {
        double g = (double)oracle_f16_to_f32(gate[qh * D + d]);
        acc *= 1.0 / (1.0 + exp(-g));
      }
      out[qh * D + d] = acc;
    }
  }
  free(s);
}

ORACLE_API void oracle_attn_causal_n_f64(const uint16_t* q,
                                         const uint16_t* gate,
                                         const uint16_t* k_rows,
                                         const uint16_t* v_rows, int64_t H,
                                         int64_t G, int64_t D,
                                         int64_t past_pos, int64_t n,
                                         double* out) {
  for (int64_t i = 0; i < n; i++)
    oracle_attn_decode_f64(q + i * H * D, gate ? gate + i * H * D : NULL, k_rows,
                           v_rows, H, G, D, past_pos + i + 1, out + i * H * D);
}

/* ------------------------------------------------ Q/K head norm + RoPE -- */

/* bf16 bit pattern -> f32 (exact). */
ORACLE_API float oracle_bf16_to_f32(uint16_t b) {
  uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* RoPE inverse frequencies as the reference computes them in f32:
 * rope_theta.powf(-2.0 * i / rotary_dim), i < rotary_dim / 2
 * (src/math_util.rs:524, 531). */
ORACLE_API void oracle_rope_inv_freq(float rope_theta, int64_t rotary_dim, float* out) {
  for (int64_t i = 0; i < rotary_dim / 2; i++)
    out[i] = powf(rope_theta, -2.0f * (float)i / (float)rotary_dim);
}

/* src/math_util.rs:501-547  q_head_norm_rope.  q_proj: [H][2*D] f32
 * (query | gate per head); q_norm_w: bf16[D]; q_out, q_gate_out: [H][D]. */
ORACLE_API void oracle_q_head_norm_rope(const float* q_proj, const uint16_t* q_norm_w,
                                        float* q_out, float* q_gate_out, int64_t num_q_heads,
                                        int64_t head_dim, int64_t rotary_dim, float rope_theta,
                                        int64_t pos, float eps) {
  int64_t rot_half = rotary_dim / 2;
  for (int64_t h = 0; h < num_q_heads; h++) {
    int64_t src_base = h * 2 * head_dim, out_base = h * head_dim;
    for (int64_t d = 0; d < head_dim; d++) q_gate_out[out_base + d] = q_proj[src_base + head_dim + d];
    float sum_sq = 0.0f;
    for (int64_t d = 0; d < head_dim; d++) { float v = q_proj[src_base + d]; sum_sq += v * v; }
    float inv_rms = 1.0f / sqrtf(sum_sq / (float)head_dim + eps);
    for (int64_t d = 0; d < head_dim; d++) {
      float q_val = q_proj[src_base + d] * inv_rms * oracle_bf16_to_f32(q_norm_w[d]);
      if (d < rotary_dim) {
        float cos_t, sin_t, pair_val;
        if (d < rot_half) {
          float theta = (float)pos * powf(rope_theta, -2.0f * (float)d / (float)rotary_dim);
          pair_val = q_proj[src_base + d + rot_half] * inv_rms * oracle_bf16_to_f32(q_norm_w[d + rot_half]);
          cos_t = cosf(theta); sin_t = sinf(theta);
          q_out[out_base + d] = q_val * cos_t - pair_val * sin_t;
        } else {
          int64_t pair = d - rot_half;
          float theta = (float)pos * powf(rope_theta, -2.0f * (float)pair / (float)rotary_dim);
          pair_val = q_proj[src_base + pair] * inv_rms * oracle_bf16_to_f32(q_norm_w[pair]);
          cos_t = cosf(theta); sin_t = sinf(theta);
          q_out[out_base + d] = pair_val * sin_t + q_val * cos_t;
        }
      } else {
        q_out[out_base + d] = q_val;
      }
    }
  }
}

/* src/math_util.rs:553-593  k_head_norm_rope (in place on k_buf [G][D]). */
ORACLE_API void oracle_k_head_norm_rope(float* k_buf, const uint16_t* k_norm_w,
                                        int64_t num_kv_heads, int64_t head_dim,
                                        int64_t rotary_dim, float rope_theta, int64_t pos,
                                        float eps) {
  int64_t rot_half = rotary_dim / 2;
  float* orig = (float*)malloc(sizeof(float) * (size_t)head_dim);
  for (int64_t h = 0; h < num_kv_heads; h++) {
    int64_t base = h * head_dim;
    float sum_sq = 0.0f;
    for (int64_t d = 0; d < head_dim; d++) { float v = k_buf[base + d]; sum_sq += v * v; }
    float inv_rms = 1.0f / sqrtf(sum_sq / (float)head_dim + eps);
    for (int64_t d = 0; d < head_dim; d++) orig[d] = k_buf[base + d];
    for (int64_t d = 0; d < head_dim; d++) {
      float k_val = orig[d] * inv_rms * oracle_bf16_to_f32(k_norm_w[d]);
      if (d < rotary_dim) {
        if (d < rot_half) {
          float theta = (float)pos * powf(rope_theta, -2.0f * (float)d / (float)rotary_dim);
          float pair_val = orig[d + rot_half] * inv_rms * oracle_bf16_to_f32(k_norm_w[d + rot_half]);
          k_buf[base + d] = k_val * cosf(theta) - pair_val * sinf(theta);
        } else {
          int64_t pair = d - rot_half;
          float theta = (float)pos * powf(rope_theta, -2.0f * (float)pair / (float)rotary_dim);
          float pair_val = orig[pair] * inv_rms * oracle_bf16_to_f32(k_norm_w[pair]);
          k_buf[base + d] = pair_val * sinf(theta) + k_val * cosf(theta);
        }
      } else {
        k_buf[base + d] = k_val;
      }
    }
  }
  free(orig);
}

/* ----------------------------------------------------- o_proj matvec -- */

/* src/engine/shaders.metal:2392-2425  matvec_bf16: out[r] = sum_c
 * bf16(W[r][c]) * x[c] (the Metal kernel's per-lane partial sums and
 * simd_sum are a reordering of this sum; here it runs in column order). */
ORACLE_API void oracle_matvec_bf16(const uint16_t* w, const float* x, float* out,
                                   int64_t out_dim, int64_t in_dim) {
  for (int64_t r = 0; r < out_dim; r++) {
    float acc = 0.0f;
    for (int64_t c = 0; c < in_dim; c++) acc += oracle_bf16_to_f32(w[r * in_dim + c]) * x[c];
    out[r] = acc;
  }
}

/* src/math_util.rs:14-57  dequant_matvec_4bit: 8 nibbles per u32 (low nibble
 * first), w = nibble * scale + bias per group of group_size columns, scales
 * and biases bf16 [out_dim][in_dim / group_size]. */
ORACLE_API void oracle_dequant_matvec_4bit(const uint32_t* w_packed, const uint16_t* scales,
                                           const uint16_t* biases, const float* x, float* out,
                                           int64_t out_dim, int64_t in_dim,
                                           int64_t group_size) {
  int64_t num_groups = in_dim / group_size;
  int64_t packed_per_group = group_size / 8;
  int64_t packed_cols = in_dim / 8;
  for (int64_t row = 0; row < out_dim; row++) {
    float acc = 0.0f;
    const uint32_t* w_row = w_packed + row * packed_cols;
    const uint16_t* s_row = scales + row * num_groups;
    const uint16_t* b_row = biases + row * num_groups;
    for (int64_t g = 0; g < num_groups; g++) {
      float scale = oracle_bf16_to_f32(s_row[g]);
      float bias = oracle_bf16_to_f32(b_row[g]);
      int64_t base_packed = g * packed_per_group;
      int64_t base_x = g * group_size;
      for (int64_t p = 0; p < packed_per_group; p++) {
        uint32_t packed = w_row[base_packed + p];
        int64_t x_base = base_x + p * 8;
        for (int n = 0; n < 8; n++) {
          uint32_t nibble = (packed >> (n * 4)) & 0xFu;
          float w_val = (float)nibble * scale + bias;
          acc += w_val * x[x_base + n];
        }
      }
    }
    out[row] = acc;
  }
}
