// mk_probe.hip — MFMA throughput ceiling of the device, measured live.
//
// The published bf16 peak (2.5 PFLOP/s dense) assumes the 2.4 GHz peak engine
// clock.  Under sustained MFMA load with random data the clock is set by the
// board's power limit instead, so the GEMM roofline is also reported against
// what the matrix cores sustain here: every CU runs one 8-wave workgroup
// (two waves per SIMD, as the GEMM does), each wave issuing independent
// v_mfma_f32_32x32x16_bf16 on 8 accumulator blocks (the GEMM's 128 fp32
// accumulators per lane) with bf16 N(0,1)-like operands that differ between
// consecutive instructions, so the multipliers toggle as they do on real
// data.  No memory traffic and no LDS: the result is the MFMA ceiling at the
// clock the power limit allows.  Wave 0 of each workgroup also samples the
// shader clock counter (s_memtime) and the constant-rate counter
// (s_memrealtime, 100 MHz) around the loop, which gives the clock the
// matrix cores ran at.
#include "mk_device.h"
#include "mk_internal.h"

namespace mk {

namespace {

constexpr int kProbeWaves = 8;
constexpr int kProbeThreads = 64 * kProbeWaves;

// Deterministic pseudo-random bf16 in about [-2, 2): a 32-bit integer hash
// (the "lowbias32" mixer) of (seed, lane, index) scaled to a float.
__device__ __forceinline__ __bf16 rnd_bf16(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return (__bf16)((float)(int32_t)x * (2.0f / 2147483648.0f));
}

__global__ __launch_bounds__(kProbeThreads, 1) void mfma_ceiling_kernel(int64_t iters, uint32_t seed, float* sink,
                                                                        uint64_t* clocks) {
  constexpr int FM = 4, FN = 2;  // 4 x 2 blocks of 32 x 32: the GEMM's wave tile of 128 x 64
  const uint32_t tid = threadIdx.x;
  const uint32_t salt = seed * 0x9e3779b9u + (blockIdx.x * kProbeThreads + tid) * 64u;
  bf16x8 a[2][FM], b[2][FN];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) a[kk][i][e] = rnd_bf16(salt + (kk * FM + i) * 8 + e);
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) b[kk][j][e] = rnd_bf16(salt + 32u + (kk * FN + j) * 8 + e + 1000003u);
  }
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  __syncthreads();
  uint64_t t0 = 0, r0 = 0;
  if (tid == 0) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[kk][j], a[kk][i], acc[i][j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) s += acc[i][j][v];
  sink[(int64_t)blockIdx.x * kProbeThreads + tid] = s;
  __syncthreads();
  if (tid == 0) {
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    clocks[blockIdx.x * 2 + 0] = t1 - t0;
    clocks[blockIdx.x * 2 + 1] = r1 - r0;
  }
}

}  // namespace

hipError_t launch_mfma_ceiling(int64_t iters, int n_wg, uint32_t seed, float* sink, uint64_t* clocks,
                               hipStream_t stream) {
  hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(n_wg), dim3(kProbeThreads), 0, stream, iters, seed, sink, clocks);
  return hipGetLastError();
}

int probe_threads() { return kProbeThreads; }

}  // namespace mk
