// plh_bench -- native driver of the C ABI (include/persistent_lstm_hip.h), without Python or torch.
//
// It builds a synthetic model (weights ~ U(-1/sqrt(H), 1/sqrt(H)) as PyTorch's default init,
// x ~ N(0, 1)), packs it with plh_pack_regressor and times plh_forward with HIP events.  It is the
// program profilers attach to (rocprofv3 -- plh_bench ...) and a worked example of the C ABI for a
// non-Python host.  Values differ from bench.py's torch-seeded ones; the kernel's work does not
// depend on them.
//
//   plh_bench [--input 5] [--hidden 128] [--layers 4] [--output 24] [--batch 512] [--seq 1000]
//             [--warmup 10] [--iters 100] [--ragged MIN] [--copy-mb N]
//   plh_bench --gemm K [--cols N] [--batch 512] [--seq 1000] [--blocked 1] [--warmup 10] [--iters 100]
//   plh_bench --issue
//
// --copy-mb N ends the run with three device-to-device copies of N MiB: a plain copy kernel of
// known size, whose memory counters calibrate the forward's HBM traffic in a profiler.
// --gemm K times plh_input_projection alone: [batch * seq, K] x [K, N] (N = --cols, default 4 K),
// fragment-blocked by default (the layer-sequential path's layout), random fp16 operands.
// --issue prints the SIMD issue rates of MFMA, v_exp_f32 and v_fma_f32 (alone, beside each other in
// the two waves of a SIMD, and interleaved in one wave), from a probe kernel of this program.
// Every run releases what it created (buffers, events, stream) before it returns.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/persistent_lstm_hip.h"

namespace {

#define HIP_OK(expr)                                                                         \
  do {                                                                                       \
    hipError_t e_ = (expr);                                                                  \
    if (e_ != hipSuccess) {                                                                  \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #expr, hipGetErrorString(e_)); \
      std::exit(1);                                                                          \
    }                                                                                        \
  } while (0)

#define PLH_OK_(expr)                                                                    \
  do {                                                                                   \
    int rc_ = (expr);                                                                    \
    if (rc_ != PLH_OK) {                                                                 \
      std::fprintf(stderr, "%s failed (%d): %s\n", #expr, rc_, plh_last_error());       \
      std::exit(1);                                                                      \
    }                                                                                    \
  } while (0)

struct Rng {  // xorshift64*
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed * 2685821657736338717ull + 1) {}
  uint64_t next() {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 2685821657736338717ull;
  }
  double uniform() { return (next() >> 11) * (1.0 / 9007199254740992.0); }
  double normal() {  // Box-Muller
    double u = uniform(), v = uniform();
    if (u < 1e-300) u = 1e-300;
    return std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v);
  }
};

std::vector<_Float16> uniform_f16(size_t n, double k, Rng& r) {
  std::vector<_Float16> v(n);
  for (auto& e : v) e = (_Float16)((2.0 * r.uniform() - 1.0) * k);
  return v;
}

void* to_device(const void* src, size_t bytes) {
  void* d = nullptr;
  HIP_OK(hipMalloc(&d, bytes ? bytes : 1));
  if (bytes) HIP_OK(hipMemcpy(d, src, bytes, hipMemcpyHostToDevice));
  return d;
}

int arg_int(int argc, char** argv, const char* name, int dflt) {
  for (int i = 1; i + 1 < argc; ++i)
    if (std::strcmp(argv[i], name) == 0) return std::atoi(argv[i + 1]);
  return dflt;
}

}  // namespace

// --gemm: the time-parallel input-projection GEMM alone.
int gemm_main(int argc, char** argv) {
  const int K = arg_int(argc, argv, "--gemm", 128), N = arg_int(argc, argv, "--cols", 4 * K);
  const long long M = (long long)arg_int(argc, argv, "--batch", 512) * arg_int(argc, argv, "--seq", 1000);
  const int blocked = arg_int(argc, argv, "--blocked", 1);
  const int warmup = arg_int(argc, argv, "--warmup", 10), iters = arg_int(argc, argv, "--iters", 100);
  const int copy_mb = arg_int(argc, argv, "--copy-mb", 0);
  Rng rng(7);
  std::vector<_Float16> w((size_t)N * K);
  for (auto& e : w) e = (_Float16)(rng.normal() / 16.0);
  void* d_w = to_device(w.data(), w.size() * 2);
  std::vector<_Float16> xrow((size_t)1 << 20);
  for (auto& e : xrow) e = (_Float16)rng.normal();
  void *d_x = nullptr, *d_c = nullptr;
  HIP_OK(hipMalloc(&d_x, (size_t)M * K * 2));
  HIP_OK(hipMalloc(&d_c, (size_t)M * N * 2));
  for (size_t off = 0; off < (size_t)M * K; off += xrow.size())
    HIP_OK(hipMemcpy((_Float16*)d_x + off, xrow.data(), std::min(xrow.size(), (size_t)M * K - off) * 2,
                     hipMemcpyHostToDevice));
  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  auto run = [&]() { PLH_OK_(plh_input_projection(d_x, K, d_w, K, d_c, N, M, N, blocked, s)); };
  for (int i = 0; i < warmup; ++i) run();
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));
  HIP_OK(hipEventRecord(e0, s));
  for (int i = 0; i < iters; ++i) run();
  HIP_OK(hipEventRecord(e1, s));
  HIP_OK(hipEventSynchronize(e1));
  float total_ms = 0.f;
  HIP_OK(hipEventElapsedTime(&total_ms, e0, e1));
  if (copy_mb > 0) {
    void *src = nullptr, *dst = nullptr;
    const size_t bytes = (size_t)copy_mb << 20;
    HIP_OK(hipMalloc(&src, bytes));
    HIP_OK(hipMalloc(&dst, bytes));
    HIP_OK(hipMemsetAsync(src, 1, bytes, s));
    for (int i = 0; i < 3; ++i) HIP_OK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s));
    HIP_OK(hipStreamSynchronize(s));
    HIP_OK(hipFree(src));
    HIP_OK(hipFree(dst));
  }
  const double ms = total_ms / iters, flops = 2.0 * (double)M * N * K;
  std::printf("{\"gemm\": [%lld, %d, %d], \"blocked\": %d, \"iters\": %d, \"ms\": %.6f, \"tflops\": %.3f}\n", M, K, N,
              blocked, iters, ms, flops / (ms * 1e-3) / 1e12);
  std::fflush(stdout);
  HIP_OK(hipEventDestroy(e0));
  HIP_OK(hipEventDestroy(e1));
  HIP_OK(hipStreamDestroy(s));
  for (void* p : {d_w, d_x, d_c}) HIP_OK(hipFree(p));
  HIP_OK(hipDeviceSynchronize());
  return 0;
}

// --issue: SIMD issue rates (plh_issue_probe.hip, built into this program only).
int plh_bench_issue_rates();

int main(int argc, char** argv) {
  for (int i = 1; i < argc; ++i) {
    if (std::strcmp(argv[i], "--gemm") == 0) return gemm_main(argc, argv);
    if (std::strcmp(argv[i], "--issue") == 0) return plh_bench_issue_rates();
  }
  const int I = arg_int(argc, argv, "--input", 5), H = arg_int(argc, argv, "--hidden", 128);
  const int L = arg_int(argc, argv, "--layers", 4), O = arg_int(argc, argv, "--output", 24);
  const int B = arg_int(argc, argv, "--batch", 512), T = arg_int(argc, argv, "--seq", 1000);
  const int warmup = arg_int(argc, argv, "--warmup", 10), iters = arg_int(argc, argv, "--iters", 100);
  const int ragged_min = arg_int(argc, argv, "--ragged", 0);
  const int copy_mb = arg_int(argc, argv, "--copy-mb", 0);
  if (!plh_supports(I, H, L, O)) {
    std::fprintf(stderr, "unsupported geometry: %s\n", plh_last_error());
    return 1;
  }
  Rng rng(42);
  const double k = 1.0 / std::sqrt((double)H);
  std::vector<void*> w_ih(L), w_hh(L), b_ih(L), b_hh(L);
  for (int l = 0; l < L; ++l) {
    const int K = l == 0 ? I : H;
    auto a = uniform_f16((size_t)4 * H * K, k, rng), b = uniform_f16((size_t)4 * H * H, k, rng);
    auto c = uniform_f16((size_t)4 * H, k, rng), d = uniform_f16((size_t)4 * H, k, rng);
    w_ih[l] = to_device(a.data(), a.size() * 2);
    w_hh[l] = to_device(b.data(), b.size() * 2);
    b_ih[l] = to_device(c.data(), c.size() * 2);
    b_hh[l] = to_device(d.data(), d.size() * 2);
  }
  auto lw = uniform_f16((size_t)O * H, k, rng), lb = uniform_f16((size_t)O, k, rng);
  void* d_lw = to_device(lw.data(), lw.size() * 2);
  void* d_lb = to_device(lb.data(), lb.size() * 2);
  std::vector<_Float16> x((size_t)B * T * I);
  for (auto& e : x) e = (_Float16)rng.normal();
  void* d_x = to_device(x.data(), x.size() * 2);
  int32_t* d_len = nullptr;
  double seq_steps = (double)B * T;
  if (ragged_min > 0) {
    std::vector<int32_t> len(B);
    for (auto& e : len) e = ragged_min + (int32_t)(rng.next() % (uint64_t)(T - ragged_min + 1));
    std::sort(len.begin(), len.end(), [](int a, int b) { return a > b; });
    seq_steps = 0;
    for (int e : len) seq_steps += e;
    d_len = (int32_t*)to_device(len.data(), len.size() * 4);
  }

  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  const int64_t pbytes = plh_packed_bytes(I, H, L, O);
  void* packed = nullptr;
  HIP_OK(hipMalloc(&packed, pbytes));
  PLH_OK_(plh_pack_regressor(I, H, L, O, w_ih.data(), w_hh.data(), b_ih.data(), b_hh.data(), d_lw, d_lb, packed,
                             pbytes, s));
  const int64_t wbytes = plh_workspace_bytes(I, H, L, O, B, T);
  void *ws = nullptr, *out = nullptr;
  HIP_OK(hipMalloc(&ws, wbytes));
  HIP_OK(hipMalloc(&out, (size_t)B * O * 2));
  auto fwd = [&]() {
    PLH_OK_(plh_forward(packed, I, H, L, O, d_x, B, T, d_len, nullptr, nullptr, out, nullptr, nullptr, nullptr,
                        nullptr, 0, nullptr, nullptr, ws, wbytes, s));
  };
  for (int i = 0; i < warmup; ++i) fwd();
  HIP_OK(hipStreamSynchronize(s));
  PLH_OK_(plh_kernel_timing(iters));
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));
  HIP_OK(hipEventRecord(e0, s));
  for (int i = 0; i < iters; ++i) fwd();
  HIP_OK(hipEventRecord(e1, s));
  HIP_OK(hipEventSynchronize(e1));
  float total_ms = 0.f;
  HIP_OK(hipEventElapsedTime(&total_ms, e0, e1));
  double kernel_ms = 0.0;
  int timed = 0;
  PLH_OK_(plh_kernel_timing_read(&kernel_ms, &timed));
  PLH_OK_(plh_kernel_timing(0));
  uint32_t status = 0;
  PLH_OK_(plh_status(ws, &status, s));
  std::vector<_Float16> host_out((size_t)B * O);
  HIP_OK(hipMemcpy(host_out.data(), out, host_out.size() * 2, hipMemcpyDeviceToHost));
  double checksum = 0.0;
  for (auto v : host_out) checksum += std::fabs((double)v);
  if (copy_mb > 0) {
    void *src = nullptr, *dst = nullptr;
    const size_t bytes = (size_t)copy_mb << 20;
    HIP_OK(hipMalloc(&src, bytes));
    HIP_OK(hipMalloc(&dst, bytes));
    HIP_OK(hipMemsetAsync(src, 1, bytes, s));
    for (int i = 0; i < 3; ++i) HIP_OK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s));
    HIP_OK(hipStreamSynchronize(s));
    HIP_OK(hipFree(src));
    HIP_OK(hipFree(dst));
  }
  const double fwd_ms = total_ms / iters, kern_ms = kernel_ms / std::max(timed, 1);
  std::printf(
      "{\"geometry\": [%d, %d, %d, %d], \"batch\": %d, \"seq\": %d, \"iters\": %d, \"fwd_ms\": %.6f, "
      "\"kernel_ms\": %.6f, \"seq_steps_per_s\": %.6e, \"status\": %u, \"abs_checksum\": %.6f}\n",
      I, H, L, O, B, T, iters, fwd_ms, kern_ms, seq_steps / (fwd_ms * 1e-3), status, checksum);
  std::fflush(stdout);
  HIP_OK(hipEventDestroy(e0));
  HIP_OK(hipEventDestroy(e1));
  HIP_OK(hipStreamDestroy(s));
  for (int l = 0; l < L; ++l)
    for (void* p : {w_ih[l], w_hh[l], b_ih[l], b_hh[l]}) HIP_OK(hipFree(p));
  for (void* p : {d_lw, d_lb, d_x, packed, ws, out}) HIP_OK(hipFree(p));
  if (d_len) HIP_OK(hipFree(d_len));
  HIP_OK(hipDeviceSynchronize());
  return status == 0 ? 0 : 2;
}
