// Measurement helpers for bench.py: bf16 MFMA throughput loops (no
// counterpart in the reference). Each wave keeps 16 independent accumulator
// chains of v_mfma_f32_16x16x32_bf16, so the matrix pipe never waits on a
// result; the accumulators are reduced into one float per thread so the work
// is kept.
//   mfma_loop_k       one fixed, low-entropy operand pair (few toggling bits):
//                     the matrix pipe's issue rate.
//   mfma_loop_rand_k  eight operand pairs of random bf16 values (uniform in
//                     [-1, 1), a hash of the lane and slot) taken in turn, two
//                     waves per SIMD (512-thread blocks, one per CU), the
//                     occupancy of the attention kernels: the rate the pipe
//                     sustains on data that toggles like real operands, which
//                     the chip's power management holds well below the issue
//                     rate.

#include "kat_common.h"
#include "kat_internal.h"

namespace kat {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void mfma_loop_k(float* __restrict__ out, int iters) {
  const int tid = threadIdx.x;
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (__bf16)(0.001f * (float)((tid + e) & 7));
    b[e] = (__bf16)(0.001f * (float)((tid * 3 + e) & 7));
  }
  f32x4 acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += (acc[i][0] + acc[i][1]) + (acc[i][2] + acc[i][3]);
  out[(size_t)blockIdx.x * blockDim.x + tid] = s;
}

__device__ __forceinline__ unsigned mix32(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

__global__ __launch_bounds__(512) void mfma_loop_rand_k(float* __restrict__ out, int iters) {
  const int tid = threadIdx.x;
  bf16x8 x[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      x[s][e] = (__bf16)((float)((int)(mix32((unsigned)(blockIdx.x * 512 + tid) * 64u + 8u * s + e) & 0xffffu) - 32768) *
                         (1.f / 32768.f));
  f32x4 acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[i & 7], x[(i + 3) & 7], acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += (acc[i][0] + acc[i][1]) + (acc[i][2] + acc[i][3]);
  out[(size_t)blockIdx.x * blockDim.x + tid] = s;
}

}  // namespace
}  // namespace kat

using namespace kat;

extern "C" int kat_probe_mfma_bf16(float* out, int blocks, int iters, double* flops, void* stream) {
  if (!out || !flops || blocks <= 0 || iters <= 0)
    return fail(KAT_EINVAL, "kat_probe_mfma_bf16: bad arguments");
  hipLaunchKernelGGL(mfma_loop_k, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), out, iters);
  // 4 waves per block, 16 MFMAs per iteration, 16 x 16 x 32 x 2 flops each
  *flops = (double)blocks * 4.0 * (double)iters * 16.0 * (16.0 * 16.0 * 32.0 * 2.0);
  return check_launch("kat_probe_mfma_bf16");
}

extern "C" int kat_probe_mfma_bf16_random(float* out, int blocks, int iters, double* flops, void* stream) {
  if (!out || !flops || blocks <= 0 || iters <= 0)
    return fail(KAT_EINVAL, "kat_probe_mfma_bf16_random: bad arguments");
  hipLaunchKernelGGL(mfma_loop_rand_k, dim3((unsigned)blocks), dim3(512), 0, as_stream(stream), out, iters);
  // 8 waves per block, 16 MFMAs per iteration, 16 x 16 x 32 x 2 flops each
  *flops = (double)blocks * 8.0 * (double)iters * 16.0 * (16.0 * 16.0 * 32.0 * 2.0);
  return check_launch("kat_probe_mfma_bf16_random");
}
