// plh_issue_probe.hip -- SIMD issue rates of MFMA, v_exp_f32 and v_fma_f32 in one or two waves of a
// SIMD: what bounds the overlap of a step's gate math with its MFMAs.  A developer measurement
// built into plh_bench (--issue) only; the product library does not contain it.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kChains = 8;  // independent chains per wave: 8 x 16 cycles covers the MFMA latency

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

// Cases: (waves 0-3, waves 4-7) roles and their names ("a|b": the two waves of a SIMD issue a and b;
// "a+b": one wave issues both, figure per pair).  Prints one JSON line per case.  Returns 0 on success.
int plh_bench_issue_rates() {
  static const int kCases[][2] = {{1, 0}, {2, 0}, {3, 0}, {1, 1}, {2, 2}, {3, 3}, {1, 2}, {1, 3}, {4, 0}, {5, 0}};
  static const char* kNames[] = {"mfma",    "exp",      "fma",      "mfma|mfma", "exp|exp",
                                 "fma|fma", "mfma|exp", "mfma|fma", "mfma+fma",  "mfma+exp"};
  constexpr int kCaseCount = sizeof(kCases) / sizeof(kCases[0]);
  float* out = nullptr;
  unsigned long long* cyc = nullptr;
  unsigned long long h[2] = {0, 0};
  hipError_t e = hipMalloc(&out, 512 * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&cyc, sizeof(h));
  for (int c = 0; c < kCaseCount && e == hipSuccess; ++c) {
    for (int rep = 0; rep < 2 && e == hipSuccess; ++rep) {  // the first run warms the clock and caches
      e = hipMemset(cyc, 0, sizeof(h));
      if (e == hipSuccess) {
        issue_probe_kernel<<<1, 512, 0, nullptr>>>(kCases[c][0], kCases[c][1], out, cyc);
        e = hipGetLastError();
      }
      if (e == hipSuccess) e = hipMemcpy(h, cyc, sizeof(h), hipMemcpyDeviceToHost);
    }
    if (e != hipSuccess) break;
    const double n_inst = kIssueIters * 8.0;
    if (std::strchr(kNames[c], '|'))
      std::printf("{\"case\": \"%s\", \"cycles_per_inst_waves_0_3\": %.2f, \"cycles_per_inst_waves_4_7\": %.2f}\n",
                  kNames[c], (double)h[0] / n_inst, (double)h[1] / n_inst);
    else
      std::printf("{\"case\": \"%s\", \"cycles_per_inst_waves_0_3\": %.2f}\n", kNames[c], (double)h[0] / n_inst);
  }
  if (out) (void)hipFree(out);
  if (cyc) (void)hipFree(cyc);
  if (e != hipSuccess) {
    std::fprintf(stderr, "issue-rate probe: %s\n", hipGetErrorString(e));
    return 1;
  }
  return 0;
}
