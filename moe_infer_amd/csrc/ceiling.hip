// MFMA issue ceiling of the device, for the prefill roofline: one wave per
// SIMD issuing v_mfma_f32_32x32x16_f16 back to back (four independent
// accumulation chains, so no MFMA waits for another), with nothing else in
// the loop: no LDS, no VALU, no memory.  The A operand rotates over eight
// register-resident fragments, so that every MFMA sees operands different
// from the previous one, as the K and V fragments of a flash-attention tile
// do.  What this kernel reaches with random operands is what the clock and
// power limits of the part leave of the nominal 2.5 PFLOP/s; the same run
// with zero operands shows how much of that is power drawn by the data.
// Each workgroup also reads its shader clock (s_memtime) against the
// constant 100 MHz counter (s_memrealtime), giving the clock the MFMA units
// ran at.
#include "common.h"

namespace {

constexpr int kFrags = 8;  // A fragments rotated through
constexpr int kChains = 4;

// One workgroup of 4 waves per CU (the LDS request keeps a second one off).
__global__ void __launch_bounds__(256, 1)
mfma_ceiling_kernel(const _Float16* ops, float* out, int iters, unsigned long long* clocks) {
  const int t = threadIdx.x;
  // per thread: kFrags A fragments and kChains B fragments of 8 halves
  const _Float16* p = ops + (size_t)t * (kFrags + kChains) * 8;
  f16x8 a[kFrags], b[kChains];
#pragma unroll
  for (int i = 0; i < kFrags; i++) a[i] = *(const f16x8*)(p + 8 * i);
#pragma unroll
  for (int j = 0; j < kChains; j++) b[j] = *(const f16x8*)(p + 8 * (kFrags + j));
  f32x16 c[kChains];
#pragma unroll
  for (int j = 0; j < kChains; j++) c[j] = f32x16{};
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int k = 0; k < kFrags; k++)
      c[k % kChains] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[k], b[k % kChains], c[k % kChains], 0, 0, 0);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kChains; j++)
#pragma unroll
    for (int e = 0; e < 16; e++) s += c[j][e];
  out[(size_t)blockIdx.x * blockDim.x + t] = s;
  if (t == 0) {
    clocks[2 * blockIdx.x] = t1 - t0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

}  // namespace

extern "C" mi_status mi_bench_mfma_ceiling(const mi_f16* operands, int32_t iters, int32_t workgroups,
                                           float* out, uint64_t* clocks, mi_stream stream) {
  mi::clear_error();
  if (!operands || !out || !clocks) return mi::fail(MI_ERR_INVALID_ARG, "null argument");
  if (iters <= 0 || workgroups <= 0)
    return mi::fail(MI_ERR_INVALID_ARG, "iters=%d workgroups=%d", iters, workgroups);
  constexpr int kLds = 96 * 1024;
  static std::atomic<uint64_t> lds_set{0};
  MI_TRY(mi::set_lds_limit((const void*)mfma_ceiling_kernel, kLds, lds_set));
  MI_HIP(mi::launch("mfma_ceiling", mfma_ceiling_kernel, dim3(workgroups), dim3(256), (size_t)kLds,
                    (hipStream_t)stream, (const _Float16*)operands, out, iters,
                    (unsigned long long*)clocks));
  return MI_OK;
}
