// clock_probe.hip - the shader clock under a matrix-core load.
//
// MI355X's datasheet bf16 peak (2.5 PFLOP/s) assumes the 2.4 GHz peak
// engine clock; under sustained MFMA load the clock the chip holds is lower.
// This kernel keeps every SIMD's matrix core busy with independent
// v_mfma_f32_32x32x16_bf16 chains and reports, per workgroup, how many
// shader-clock ticks (s_memtime) and how many constant-rate real-time ticks
// (s_memrealtime, hipDeviceAttributeWallClockRate) its loop took: their
// ratio times the real-time rate is the clock the loop ran at. A
// measurement aid for the benchmark; it reads no memory and writes two
// 64-bit words per workgroup.
#include "bd3_device.h"
#include "bd3_launch.h"

namespace bd3 {
namespace {

__global__ __launch_bounds__(256) void clock_probe_kernel(uint64_t* out, int iters) {
  // Four independent accumulator chains per wave: each MFMA's result is
  // needed only four instructions later, so the matrix core never waits.
  const float seed = (float)(wi_x() & 7) * 0x1p-10f;
  bf16x8 a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (__bf16)(seed + 0.5f);
    b[j] = (__bf16)(0.25f - seed);
  }
  f32x16 acc[4] = {};
  __syncthreads();
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t w0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = mfma32(a, b, acc[u]);
  }
  // Reading the accumulators waits for the last products; the sum feeds a
  // store that never happens, so the chains cannot be removed.
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u) s += acc[u][0] + acc[u][15];
  __syncthreads();
  const uint64_t c1 = __builtin_amdgcn_s_memtime();
  const uint64_t w1 = __builtin_amdgcn_s_memrealtime();
  if (wi_x() == 0) {
    out[2 * wg_x()] = c1 - c0;
    out[2 * wg_x() + 1] = w1 - w0;
  }
  if (s == -1.f) out[2 * wg_x()] = 0;  // never true: the products are positive
}

}  // namespace

hipError_t launch_clock_probe(uint64_t* out, int workgroups, int iters, hipStream_t stream) {
  hipLaunchKernelGGL(clock_probe_kernel, dim3((unsigned)workgroups), dim3(256), 0, stream, out, iters);
  return hipGetLastError();
}

}  // namespace bd3
