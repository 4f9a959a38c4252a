// plh_probe.hip -- on-box measurement behind the roofline figure: the dense fp16 MFMA rate the
// GPU sustains with v_mfma_f32_16x16x32_f16 (the instruction the recurrent kernels use) on every
// CU, with the shader clock during that run.  A diagnostic for the benchmark; nothing on the
// forward path calls it.
#include "plh_internal.h"

namespace plh {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kChains = 8;  // independent accumulators per wave: 8 x 16 cycles covers the MFMA latency

// One workgroup per CU: 16 waves (four per SIMD), and 96 KB of LDS reserved so that no second
// workgroup fits on a CU (small workgroups may otherwise be packed onto some CUs while others idle).
// Every wave issues iters x kChains MFMAs from register operands (lane-dependent values, so nothing
// folds) and writes its sum; thread 0 of each workgroup records the elapsed shader cycles
// (s_memtime) and 100 MHz reference ticks (s_memrealtime) of its loop.
constexpr int kProbeThreads = 1024;
__global__ void __launch_bounds__(kProbeThreads) mfma_probe_kernel(int iters, float* out, unsigned long long* clk) {
  __shared__ float reserve[24 * 1024];
  const int lane = threadIdx.x & 63;
  if (iters < 0) {  // never taken; a store and a read keep the reservation
    reserve[threadIdx.x] = 1.f;
    __syncthreads();
    out[threadIdx.x] = reserve[threadIdx.x ^ 1];
  }
  f16x8_t a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (_Float16)((lane + j) * 0.001f);
    b[j] = (_Float16)((lane - j) * 0.001f);
  }
  f32x4_t acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = t1 - t0;
    clk[2 * blockIdx.x + 1] = r1 - r0;
  }
}

}  // namespace

hipError_t launch_mfma_probe(int blocks, int iters, float* out, unsigned long long* clk, hipStream_t s) {
  mfma_probe_kernel<<<blocks, kProbeThreads, 0, s>>>(iters, out, clk);
  return hipGetLastError();
}

double mfma_probe_flops(int blocks, int iters) {
  return (double)blocks * (kProbeThreads / 64) * iters * kChains * (16.0 * 16.0 * 32.0 * 2.0);
}

}  // namespace plh
