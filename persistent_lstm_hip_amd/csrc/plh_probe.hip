// plh_probe.hip -- on-box measurements behind the roofline figures: the dense fp16 MFMA rate the
// GPU sustains with v_mfma_f32_16x16x32_f16 (the instruction the recurrent kernels use) on every
// CU with the shader clock during that run, and the issue rates of MFMA, v_exp_f32 and v_fma_f32
// in one or two waves of a SIMD (what bounds the overlap of a step's gate math with its MFMAs).
// Diagnostics for the benchmark; nothing on the forward path calls them.
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

// Issue-rate probe: one workgroup of 8 waves (two per SIMD: waves w and w + 4 share SIMD w), waves
// 0-3 running role `ra` and waves 4-7 role `rb`, each for kIssueIters x 8 instructions of its kind from
// 8 independent chains; lane 0 of waves 0 and 4 records the elapsed shader cycles (s_memtime).
// Roles: 0 idle, 1 v_mfma_f32_16x16x32_f16, 2 v_exp_f32 (of -|x|, so values stay finite),
// 3 v_fma_f32, 4 an MFMA and an FMA of independent chains, 5 an MFMA and an exp.
constexpr int kIssueIters = 512;  // x 8 instructions per wave; compile-time, so the loops unroll (x4)
__device__ __forceinline__ unsigned long long issue_role(int role, float seed, float* sink) {
  const int lane = threadIdx.x & 63;
  f16x8_t a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (_Float16)((lane + j) * 0.001f * seed);
    b[j] = (_Float16)((lane - j) * 0.001f);
  }
  f32x4_t acc[kChains];
  float e[kChains], g[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) {
    acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    e[c] = seed * 1e-3f + lane * 1e-6f + c * 1e-4f;
    g[c] = seed + lane * 1e-3f + c;
  }
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  if (role == 1) {
#pragma unroll 4
    for (int it = 0; it < kIssueIters; ++it)
#pragma unroll
      for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
  } else if (role == 2) {
#pragma unroll 4
    for (int it = 0; it < kIssueIters; ++it)
#pragma unroll
      for (int c = 0; c < kChains; ++c) e[c] = __builtin_amdgcn_exp2f(-__builtin_fabsf(e[c]));
  } else if (role == 3) {
#pragma unroll 4
    for (int it = 0; it < kIssueIters; ++it)
#pragma unroll
      for (int c = 0; c < kChains; ++c) g[c] = __builtin_fmaf(g[c], 0.999f, 0.001f);
  } else if (role == 4) {
#pragma unroll 4
    for (int it = 0; it < kIssueIters; ++it)
#pragma unroll
      for (int c = 0; c < kChains; ++c) {
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
        g[c] = __builtin_fmaf(g[c], 0.999f, 0.001f);
      }
  } else if (role == 5) {
#pragma unroll 4
    for (int it = 0; it < kIssueIters; ++it)
#pragma unroll
      for (int c = 0; c < kChains; ++c) {
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
        e[c] = __builtin_amdgcn_exp2f(-__builtin_fabsf(e[c]));
      }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += acc[c][0] + acc[c][3] + e[c] + g[c];
  *sink = s;
  return t1 - t0;
}

__global__ void __launch_bounds__(512) issue_probe_kernel(int ra, int rb, float* out, unsigned long long* cyc) {
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const unsigned long long d = issue_role(wave < 4 ? ra : rb, 1.0f, out + threadIdx.x);
  if ((threadIdx.x & 63) == 0 && (wave == 0 || wave == 4)) cyc[wave >> 2] = d;
}

}  // namespace

hipError_t launch_issue_probe(int ra, int rb, float* out, unsigned long long* cyc, hipStream_t s) {
  issue_probe_kernel<<<1, 512, 0, s>>>(ra, rb, out, cyc);
  return hipGetLastError();
}

int issue_probe_instructions() { return kIssueIters * 8; }

hipError_t launch_mfma_probe(int blocks, int iters, float* out, unsigned long long* clk, hipStream_t s) {
  mfma_probe_kernel<<<blocks, kProbeThreads, 0, s>>>(iters, out, clk);
  return hipGetLastError();
}

double mfma_probe_flops(int blocks, int iters) {
  return (double)blocks * (kProbeThreads / 64) * iters * kChains * (16.0 * 16.0 * 32.0 * 2.0);
}

}  // namespace plh
