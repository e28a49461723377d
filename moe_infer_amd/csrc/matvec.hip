// o_proj of the attention output: out[r] = sum_c W[r][c] * x[c], with W in
// bf16 (the BQ4 layout of the attention projections) or in the reference's
// 4-bit affine format (8 nibbles per u32, low nibble first; per group of
// group_size columns w = nibble * scale + bias, scales and biases bf16).
//
// Reference semantics: matvec_bf16 (src/engine/shaders.metal:2392-2425) and
// dequant_matvec_4bit (src/math_util.rs:14-57), dispatched for the o_proj by
// encode_matvec_into (src/engine/qwen35_moe/fused_exp2.rs:732; metal_context.rs
// 959-980) after the sigmoid gate.
//
// HBM bound: W is read once (16 MiB in bf16, 4 MiB + 0.5 MiB in 4-bit for
// 2048 x 4096).  One wavefront per row (bf16) or per two rows (4-bit, the
// pieces of x reused for both); every lane streams 16-byte pieces of its
// rows with the matching pieces of x, all loads issued before the first
// FMA; the row sum is a DPP wave reduction.  x is the f16 attention output.
// Rows per wave, measured at 2048 x 4096 over 40 / 96 cold matrices (kernel
// us): bf16 1 row 4.2, 2 rows 4.7, 4 rows 5.9; 4-bit 2 rows 4.1, 1 row 4.1,
// 4 rows 4.8; 8 waves per workgroup instead of 4 was no faster.
#include "common.h"

extern "C" __device__ float __ockl_wfred_add_f32(float);

namespace {

constexpr int kBf16Rows = 1;  // rows per wave, bf16 kernel
constexpr int kQ4Rows = 2;    // rows per wave, 4-bit kernel
constexpr int kWaves = 4;

__device__ __forceinline__ u32x4 load_nt(const void* p) {
  return __builtin_nontemporal_load((const u32x4*)p);
}

// bf16 weights: chunk k of a row = columns 512k .. 512k + 511, lane l holds
// columns 512k + 8l .. +7.  KB chunks are loaded per batch.
__global__ void __launch_bounds__(kWaves * 64)
matvec_bf16_kernel(const _Float16* __restrict__ x, const uint16_t* __restrict__ w,
                   float* __restrict__ out, int out_dim, int in_dim) {
  constexpr int KB = 8;
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * kBf16Rows;
  if (row0 >= out_dim) return;  // whole waves
  const int nk = in_dim / 512;
  float acc[kBf16Rows] = {};
  for (int kb = 0; kb < nk; kb += KB) {
    f16x8 xv[KB];
    u32x4 wv[kBf16Rows][KB];
#pragma unroll
    for (int k = 0; k < KB; k++) {
      if (kb + k < nk) {
        const int c0 = 512 * (kb + k) + 8 * lane;
        xv[k] = *(const f16x8*)(x + c0);
#pragma unroll
        for (int r = 0; r < kBf16Rows; r++) {
          const int row = min(row0 + r, out_dim - 1);
          wv[r][k] = load_nt(w + (int64_t)row * in_dim + c0);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < KB; k++) {
      if (kb + k < nk) {
#pragma unroll
        for (int r = 0; r < kBf16Rows; r++) {
          const uint32_t ww[4] = {wv[r][k].x, wv[r][k].y, wv[r][k].z, wv[r][k].w};
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const uint16_t b = (uint16_t)(ww[e >> 1] >> (16 * (e & 1)));
            acc[r] = fmaf(mi::bf16_to_f32(b), (float)xv[k][e], acc[r]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kBf16Rows; r++) {
    const float s = __ockl_wfred_add_f32(acc[r]);
    if (lane == 0 && row0 + r < out_dim) out[row0 + r] = s;
  }
}

// 4-bit weights: chunk k of a row = columns 2048k .. 2048k + 2047 = packed
// words 256k .. 256k + 255; lane l holds words 256k + 4l .. +3 = columns
// 2048k + 32l .. +31, all inside one group (group_size is a multiple of 32).
__global__ void __launch_bounds__(kWaves * 64)
matvec_q4_kernel(const _Float16* __restrict__ x, const uint32_t* __restrict__ wp,
                 const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
                 float* __restrict__ out, int out_dim, int in_dim, int group_size) {
  constexpr int KB = 4;
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * kQ4Rows;
  if (row0 >= out_dim) return;  // whole waves
  const int nk = in_dim / 2048;
  const int ngroups = in_dim / group_size;
  float acc[kQ4Rows] = {0.f, 0.f};
  for (int kb = 0; kb < nk; kb += KB) {
    u32x4 wv[kQ4Rows][KB];
    float sc[kQ4Rows][KB], bi[kQ4Rows][KB];
    f16x8 xv[KB][4];
#pragma unroll
    for (int k = 0; k < KB; k++) {
      if (kb + k < nk) {
        const int c0 = 2048 * (kb + k) + 32 * lane;
#pragma unroll
        for (int q = 0; q < 4; q++) xv[k][q] = *(const f16x8*)(x + c0 + 8 * q);
        const int g = c0 / group_size;
#pragma unroll
        for (int r = 0; r < kQ4Rows; r++) {
          const int row = min(row0 + r, out_dim - 1);
          wv[r][k] = load_nt(wp + (int64_t)row * (in_dim / 8) + c0 / 8);
          sc[r][k] = mi::bf16_to_f32(scales[(int64_t)row * ngroups + g]);
          bi[r][k] = mi::bf16_to_f32(biases[(int64_t)row * ngroups + g]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < KB; k++) {
      if (kb + k < nk) {
#pragma unroll
        for (int r = 0; r < kQ4Rows; r++) {
          const uint32_t ww[4] = {wv[r][k].x, wv[r][k].y, wv[r][k].z, wv[r][k].w};
#pragma unroll
          for (int q = 0; q < 4; q++)
#pragma unroll
            for (int n = 0; n < 8; n++) {
              const float wval = (float)((ww[q] >> (4 * n)) & 0xFu) * sc[r][k] + bi[r][k];
              acc[r] = fmaf(wval, (float)xv[k][q][n], acc[r]);
            }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kQ4Rows; r++) {
    const float s = __ockl_wfred_add_f32(acc[r]);
    if (lane == 0 && row0 + r < out_dim) out[row0 + r] = s;
  }
}

int grid_for(int out_dim, int rows_per_wave) {
  const int rows_per_wg = kWaves * rows_per_wave;
  return (out_dim + rows_per_wg - 1) / rows_per_wg;
}

}  // namespace

extern "C" mi_status mi_matvec_bf16(const mi_f16* x, const uint16_t* w, float* out,
                                    int32_t out_dim, int32_t in_dim, mi_stream stream) {
  mi::clear_error();
  if (!x || !w || !out) return mi::fail(MI_ERR_INVALID_ARG, "null pointer");
  if (out_dim <= 0 || in_dim <= 0 || in_dim % 512)
    return mi::fail(MI_ERR_INVALID_ARG, "out_dim=%d in_dim=%d (in_dim a multiple of 512)",
                    out_dim, in_dim);
  MI_HIP(mi::launch("matvec_bf16", matvec_bf16_kernel, dim3(grid_for(out_dim, kBf16Rows)),
                    dim3(kWaves * 64), 0, (hipStream_t)stream, (const _Float16*)x, w, out,
                    out_dim, in_dim));
  return MI_OK;
}

extern "C" mi_status mi_matvec_q4(const mi_f16* x, const uint32_t* w_packed,
                                  const uint16_t* scales, const uint16_t* biases,
                                  int32_t group_size, float* out, int32_t out_dim,
                                  int32_t in_dim, mi_stream stream) {
  mi::clear_error();
  if (!x || !w_packed || !scales || !biases || !out)
    return mi::fail(MI_ERR_INVALID_ARG, "null pointer");
  if (out_dim <= 0 || in_dim <= 0 || in_dim % 2048)
    return mi::fail(MI_ERR_INVALID_ARG, "out_dim=%d in_dim=%d (in_dim a multiple of 2048)",
                    out_dim, in_dim);
  if (group_size <= 0 || group_size % 32 || in_dim % group_size)
    return mi::fail(MI_ERR_INVALID_ARG, "group_size=%d (a multiple of 32 dividing in_dim)",
                    group_size);
  MI_HIP(mi::launch("matvec_q4", matvec_q4_kernel, dim3(grid_for(out_dim, kQ4Rows)), dim3(kWaves * 64),
                    0, (hipStream_t)stream, (const _Float16*)x, w_packed, scales, biases, out,
                    out_dim, in_dim, group_size));
  return MI_OK;
}
