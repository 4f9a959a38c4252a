// plh_pack.hip -- the layout kernels of the forward: weight packing into per-lane MFMA fragments,
// x into B-fragment order, and small fills.
#include <algorithm>

#include "plh_device.h"

namespace plh {
namespace {

// ---------------------------------------------------------------------------------------------
// Weight packing: torch layout -> per-lane MFMA A fragments.
// For 16x16x32 f16, lane l of the A operand holds A[m = l % 16][k = 8 * (l / 16) + j], j < 8.
// Row m of tile (wave w, gate q) is gate column q*H + w*16 + m; K runs over [x | h] in chunks
// of 32: chunks [0, kci) index W_ih columns, [kci, kc) index W_hh columns; out-of-range -> 0.
template <int HP>
__global__ void pack_layer_kernel(const _Float16* __restrict__ w_ih, const _Float16* __restrict__ w_hh, int K,
                                  int H, _Float16* __restrict__ dst) {
  constexpr int kWaves = HP / 16, kKci = HP / 32, kKc = 2 * kKci;
  const size_t total = (size_t)kWaves * kKc * 4 * 64 * 8;
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int j = e & 7;
  const int lane = (e >> 3) & 63;
  const int q = (e >> 9) & 3;
  const int kc = (int)((e >> 11) % kKc);
  const int wv = (int)((e >> 11) / kKc);
  const int m = lane & 15, kgrp = lane >> 4;
  const int u = wv * 16 + m;
  const size_t col = (size_t)q * H + u;
  _Float16 v = (_Float16)0.0f;
  if (u < H) {
    if (kc < kKci) {
      const int k = kc * 32 + kgrp * 8 + j;
      if (k < K) v = w_ih[col * K + k];
    } else {
      const int k = (kc - kKci) * 32 + kgrp * 8 + j;
      if (k < H) v = w_hh[col * H + k];
    }
  }
  dst[e] = v;
}

// Sliced weights: [L][S][8 waves][2 KCH chunks][NJ tiles][64 lanes][8].  Wave w of slice s holds
// the gate rows of its 4 NJ units s HS + 4 NJ w + 0 .. 4 NJ - 1 over all of K: chunks 0 .. KCH - 1
// of W_ih (the layer input, zero past K), then KCH chunks of W_hh; row r of tile j is gate r % 4 of
// unit s HS + 4 NJ w + 4 j + r / 4, and lane l of chunk kc holds k = 32 kc + 8 (l / 16) + 0 .. 7.
template <int HP>
__global__ void pack_sliced_kernel(const _Float16* __restrict__ w_ih, const _Float16* __restrict__ w_hh, int K,
                                   int H, _Float16* __restrict__ dst) {
  using C = Sliced<HP>;
  constexpr int NJ = C::kNj, KCH = C::kKch;
  const size_t total = (size_t)C::kS * 8 * 2 * KCH * NJ * 64 * 8;
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int jj = e & 7;
  const int lane = (e >> 3) & 63;
  size_t rest = e >> 9;
  const int j = (int)(rest % NJ);
  rest /= NJ;
  const int kc = (int)(rest % (2 * KCH));
  rest /= 2 * KCH;
  const int wv = (int)(rest % 8);
  const int sl = (int)(rest / 8);
  const int r = lane & 15;
  const int u = sl * C::kHs + wv * 4 * NJ + 4 * j + (r >> 2);
  const size_t col = (size_t)(r & 3) * H + u;
  const int k = (kc % KCH) * 32 + (lane >> 4) * 8 + jj;
  _Float16 v = (_Float16)0.0f;
  if (u < H) {
    if (kc < KCH) {
      if (k < K) v = w_ih[col * K + k];
    } else {
      if (k < H) v = w_hh[col * H + k];
    }
  }
  dst[e] = v;
}

__global__ void pack_bias_kernel(const _Float16* __restrict__ b_ih, const _Float16* __restrict__ b_hh, int H, int HP,
                                 float* __restrict__ dst) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= 4 * HP) return;
  const int q = e / HP, u = e % HP;
  float v = 0.0f;
  if (u < H) {
    if (b_ih) v += (float)b_ih[q * H + u];
    if (b_hh) v += (float)b_hh[q * H + u];
  }
  dst[e] = v;
}

__global__ void pack_linear_kernel(const _Float16* __restrict__ w, const _Float16* __restrict__ b, int O, int H,
                                   int HP, float* __restrict__ wl, float* __restrict__ bl) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < O * HP) {
    const int o = e / HP, k = e % HP;
    wl[e] = k < H ? (float)w[(size_t)o * H + k] : 0.0f;
  }
  if (e < O) bl[e] = b ? (float)b[e] : 0.0f;
}

// Forward prologue: x of rows [row0, row_end) into xp (B-fragment order: per tile and step, g0
// 8-wide K groups of `rows` f16x8, zero past I and past row_end), and the zeroing of up to three
// u32 ranges (status, counters, exchange ring), in one launch.
__global__ void forward_prologue_kernel(const _Float16* __restrict__ x, int T, int I, int row0, int row_end,
                                        int ntile, int rows, int g0, f16x8* __restrict__ xp,
                                        uint32_t* __restrict__ z0, size_t n0, uint32_t* __restrict__ z1,
                                        size_t n1, uint32_t* __restrict__ z2, size_t n2) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < n0) z0[e] = 0u;
  if (e < n1) z1[e] = 0u;
  if (e < n2) z2[e] = 0u;
  const int per = g0 * rows;
  if (e >= (size_t)ntile * T * per) return;
  const int f = (int)(e % per);
  const size_t tt = e / per;
  const int t = (int)(tt % T);
  const int tile = (int)(tt / T);
  const int b = row0 + tile * rows + f % rows;
  const int k0 = (f / rows) * 8;
  f16x8 v = {};
  if (b < row_end) {
    const _Float16* src = x + ((size_t)b * T + t) * I;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (k0 + j < I) v[j] = src[k0 + j];
  }
  xp[e] = v;
}

__global__ void zero_u32_kernel(uint32_t* __restrict__ p, size_t n) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < n) p[e] = 0u;
}

__global__ void repeat_first_row_kernel(const _Float16* __restrict__ in, _Float16* __restrict__ out, int rows, int cols) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < (size_t)rows * cols) out[e] = in[e % cols];
}

inline unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

hipError_t launch_pack_layer(const Geometry& g, int layer, const _Float16* w_ih, const _Float16* w_hh, _Float16* wpack,
                             hipStream_t s) {
  const size_t per_layer = (size_t)(g.HP / 16) * g.kc * 4 * 64 * 8;
  _Float16* dst = wpack + per_layer * layer;
  const int K = layer == 0 ? g.I : g.H;
  const unsigned grid = blocks_for(per_layer, 256);
  switch (g.HP) {
    case 32: hipLaunchKernelGGL(pack_layer_kernel<32>, grid, 256, 0, s, w_ih, w_hh, K, g.H, dst); break;
    case 64: hipLaunchKernelGGL(pack_layer_kernel<64>, grid, 256, 0, s, w_ih, w_hh, K, g.H, dst); break;
    case 128: hipLaunchKernelGGL(pack_layer_kernel<128>, grid, 256, 0, s, w_ih, w_hh, K, g.H, dst); break;
    case 256: hipLaunchKernelGGL(pack_sliced_kernel<256>, grid, 256, 0, s, w_ih, w_hh, K, g.H, dst); break;
    case 512: hipLaunchKernelGGL(pack_sliced_kernel<512>, grid, 256, 0, s, w_ih, w_hh, K, g.H, dst); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_pack_bias(const Geometry& g, int layer, const _Float16* b_ih, const _Float16* b_hh, float* bias,
                            hipStream_t s) {
  hipLaunchKernelGGL(pack_bias_kernel, blocks_for(4 * g.HP, 256), 256, 0, s, b_ih, b_hh, g.H, g.HP,
                     bias + (size_t)layer * 4 * g.HP);
  return hipGetLastError();
}

hipError_t launch_pack_linear(const Geometry& g, const _Float16* w, const _Float16* b, float* wlin, float* blin,
                              hipStream_t s) {
  if (g.O == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_linear_kernel, blocks_for((size_t)g.O * g.HP, 256), 256, 0, s, w, b, g.O, g.H, g.HP, wlin,
                     blin);
  return hipGetLastError();
}

hipError_t launch_forward_prologue(const Geometry& g, const ForwardArgs& a, uint32_t* status, int g0,
                                   size_t ring_words, hipStream_t s) {
  const size_t npack = (size_t)a.ntile * a.T * g0 * a.tile_rows;
  const size_t nstat = status ? 1 : 0;
  const size_t nctr = (size_t)g.L * a.ntile * counter_stride(g);
  const size_t nring = ring_words * 2;  // u64 words as u32
  const size_t n = std::max(std::max(npack, nstat), std::max(nctr, nring));
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(forward_prologue_kernel, blocks_for(n, 256), 256, 0, s, a.x, a.T, a.I, a.row0, a.row_end,
                     a.ntile, a.tile_rows, g0, a.xp, status, nstat, a.counters, nctr,
                     reinterpret_cast<uint32_t*>(a.xring), nring);
  return hipGetLastError();
}

hipError_t launch_zero_u32(uint32_t* p, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(zero_u32_kernel, blocks_for(n, 256), 256, 0, s, p, n);
  return hipGetLastError();
}

hipError_t launch_repeat_first_row(const _Float16* in, _Float16* out, int rows, int cols, hipStream_t s) {
  const size_t n = (size_t)rows * cols;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(repeat_first_row_kernel, blocks_for(n, 256), 256, 0, s, in, out, rows, cols);
  return hipGetLastError();
}

}  // namespace plh
