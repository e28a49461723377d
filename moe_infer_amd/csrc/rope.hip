// Per-head RMS norm + NeoX partial rotary embedding of Q and K, fused with the
// KV-cache append of the rotated K and the raw V rows.
//
// One wavefront per head; lane l holds columns 4l..4l+3 of head_dim = 256.
// Waves 0..H-1 of a token take the query heads (q_proj block [Q | gate]),
// waves H..H+G-1 the KV heads (K norm + rope into the cache, V converted and
// stored beside it).  The RoPE partner of column d < rotary_dim/2 is
// d + rotary_dim/2, i.e. lane l + rotary_dim/8, fetched with a cross-lane
// shuffle of the normed values.
//
// Reference semantics: q_head_norm_rope / k_head_norm_rope
// (src/math_util.rs:501-593; Metal kernels src/engine/shaders.metal:2244-2363)
// followed by kv_cache_append (math_util.rs:387-392).  K is rotated from its
// un-rotated normed values (the CPU form's `orig` copy, math_util.rs:566).
#include <cmath>

#include "common.h"

namespace {

constexpr int kMaxRotHalf = MI_ROPE_MAX_DIM / 2;

struct RopeArgs {
  const float* q_proj;    // [n][H][2*D]
  const float* k;         // [n][G][D]
  const float* v;         // [n][G][D]
  const uint16_t* q_w;    // bf16 [D]
  const uint16_t* k_w;    // bf16 [D]
  _Float16* q_out;        // [n][H][D]
  _Float16* gate_out;     // [n][H][D]
  _Float16* kc;           // cache K blocks of the layer
  _Float16* vc;           // cache V blocks of the layer
  int64_t pos;            // row of token 0
  int H, G, rot_half;
  float eps;
  // rope_theta^(-2i/rotary_dim), computed on the host in f32 with the
  // reference's expression so that theta = pos * inv_freq rounds identically.
  float inv_freq[kMaxRotHalf];
};

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

__global__ void __launch_bounds__(256) qk_norm_rope_kernel(const RopeArgs a) {
  constexpr int D = mi::kHeadDim;
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int t = blockIdx.x;
  if (head >= a.H + a.G) return;  // whole waves
  const bool is_q = head < a.H;
  const int kh = head - a.H;
  const int c0 = 4 * lane;

  const float* src = is_q ? a.q_proj + ((int64_t)t * a.H + head) * (2 * D)
                          : a.k + ((int64_t)t * a.G + kh) * D;
  const float4 x = *(const float4*)(src + c0);
  const uint16_t* w = is_q ? a.q_w : a.k_w;
  const ushort4 wb = *(const ushort4*)(w + c0);

  float ss = x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
  ss = wave_sum(ss);
  const float inv_rms = 1.0f / sqrtf(ss / (float)D + a.eps);

  float y[4] = {x.x * inv_rms * mi::bf16_to_f32(wb.x), x.y * inv_rms * mi::bf16_to_f32(wb.y),
                x.z * inv_rms * mi::bf16_to_f32(wb.z), x.w * inv_rms * mi::bf16_to_f32(wb.w)};

  const int rh = a.rot_half;
  const bool lower = c0 < rh;
  const int partner = lower ? lane + (rh >> 2) : lane - (rh >> 2);
  float pr[4];
#pragma unroll
  for (int e = 0; e < 4; e++) pr[e] = __shfl(y[e], partner & 63, 64);
  if (c0 < 2 * rh) {
    const float fpos = (float)(a.pos + t);
    const int p0 = lower ? c0 : c0 - rh;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float theta = fpos * a.inv_freq[p0 + e];
      float s, c;
      sincosf(theta, &s, &c);
      y[e] = lower ? y[e] * c - pr[e] * s : pr[e] * s + y[e] * c;
    }
  }
  f16x4 h;
#pragma unroll
  for (int e = 0; e < 4; e++) h[e] = (_Float16)y[e];

  if (is_q) {
    const int64_t o = ((int64_t)t * a.H + head) * D + c0;
    *(f16x4*)(a.q_out + o) = h;
    const float4 g = *(const float4*)(src + D + c0);
    f16x4 gh;
    gh[0] = (_Float16)g.x;
    gh[1] = (_Float16)g.y;
    gh[2] = (_Float16)g.z;
    gh[3] = (_Float16)g.w;
    *(f16x4*)(a.gate_out + o) = gh;
  } else {
    const int64_t r = a.pos + t;
    *(f16x4*)(a.kc + mi::k_offset(r, kh, c0, a.G, D)) = h;
    const float4 vv = *(const float4*)(a.v + ((int64_t)t * a.G + kh) * D + c0);
    const float vs[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
    for (int e = 0; e < 4; e++) a.vc[mi::v_offset(r, kh, c0 + e, a.G, D)] = (_Float16)vs[e];
  }
}

}  // namespace

namespace mi {

mi_status check_rope(const mi_kv* kv, int32_t rotary_dim, float rope_theta, float eps) {
  if (rotary_dim < 0 || rotary_dim % 8 || rotary_dim > kv->D || rotary_dim > MI_ROPE_MAX_DIM)
    return fail(MI_ERR_INVALID_ARG, "rotary_dim=%d (multiple of 8, at most %d)", rotary_dim,
                std::min(kv->D, MI_ROPE_MAX_DIM));
  if (!(eps >= 0.f) || !(rope_theta > 0.f))
    return fail(MI_ERR_INVALID_ARG, "eps=%g rope_theta=%g", (double)eps, (double)rope_theta);
  return MI_OK;
}

void rope_inv_freq(float rope_theta, int32_t rotary_dim, float* inv_freq) {
  for (int i = 0; i < rotary_dim / 2; i++)
    inv_freq[i] = powf(rope_theta, -2.0f * (float)i / (float)rotary_dim);
}

}  // namespace mi

extern "C" mi_status mi_qk_norm_rope_append(mi_kv* kv, int32_t layer, const float* q_proj,
                                            const float* k, const float* v,
                                            const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                            int32_t rotary_dim, float rope_theta, float eps,
                                            int64_t pos, int32_t n, mi_f16* q_out,
                                            mi_f16* gate_out, mi_stream stream) {
  mi::clear_error();
  MI_TRY(mi::check_layer(kv, layer));
  if (!q_proj || !k || !v || !q_norm_w || !k_norm_w || !q_out || !gate_out)
    return mi::fail(MI_ERR_INVALID_ARG, "null pointer");
  if (n <= 0) return mi::fail(MI_ERR_INVALID_ARG, "n=%d", n);
  if (pos < 0) return mi::fail(MI_ERR_OUT_OF_RANGE, "pos=%lld", (long long)pos);
  MI_TRY(mi::check_rope(kv, rotary_dim, rope_theta, eps));
  MI_TRY(mi::kv_grow(kv, pos + n, (hipStream_t)stream));

  RopeArgs a{};
  a.q_proj = q_proj;
  a.k = k;
  a.v = v;
  a.q_w = q_norm_w;
  a.k_w = k_norm_w;
  a.q_out = (_Float16*)q_out;
  a.gate_out = (_Float16*)gate_out;
  a.kc = kv->k[layer];
  a.vc = kv->v[layer];
  a.pos = pos;
  a.H = kv->H;
  a.G = kv->G;
  a.rot_half = rotary_dim / 2;
  a.eps = eps;
  mi::rope_inv_freq(rope_theta, rotary_dim, a.inv_freq);

  const int waves = kv->H + kv->G;
  MI_HIP(mi::launch("qk_norm_rope", qk_norm_rope_kernel, dim3(n, (waves + 3) / 4), dim3(256), 0,
                    (hipStream_t)stream, a));
  kv->len[layer] = pos + n;
  return MI_OK;
}
