// plh_kernels.hip -- CDNA4 (gfx950) kernels of the stacked LSTM + Linear inference forward.
//
// The hot kernel is a persistent, weight-stationary, layer-wavefront recurrence:
//
//   * one workgroup per (layer l, batch tile of 16 rows); all L * ntile workgroups are co-resident
//     (cooperative launch) and loop over the time steps themselves;
//   * each wave owns 16 hidden units and keeps the i, f, g, o rows of [W_ih | W_hh] for them in
//     VGPRs for the whole sequence as fp16 MFMA A fragments (128 KB + 128 KB per layer at H = 128);
//   * per step a wave computes gates^T[64 gate cols, 16 rows] = W[64, K] * [in_t | h_{t-1}]^T[K, 16]
//     with v_mfma_f32_16x16x32_f16 (fp32 accumulate, bias as the initial accumulator); the gate
//     nonlinearities and the c/h update run on the accumulator registers; c never leaves VGPRs;
//   * activations live in "fragment order": a [16 rows x 32k] block is stored as [k/8][row][8],
//     i.e. exactly the B operand of one MFMA (lane l reads 16 B at l * 16).  h_t goes to LDS in that
//     order (double-buffered) for the tile's next step and, for l < L-1, to a global hand-off buffer
//     in the same order, so LDS reads/writes are conflict-free and global traffic is contiguous;
//   * the step input (x for layer 0, h^{l-1} otherwise) reaches LDS one chunk of `CH` steps at a
//     time: the chunk is loaded to VGPRs during the previous chunk and written to an LDS ring at the
//     chunk boundary, so no step waits on global memory;
//   * the hand-off between layers is a per-(layer, tile) step counter published with an agent-scope
//     release at chunk boundaries and observed with a deferred poll + agent-scope acquire one chunk
//     ahead: layer l+1 works on chunk k while layer l works on later chunks (layer wavefront);
//   * the Linear head runs in the last layer's epilogue on the final h held in LDS.
//
// Reference behaviour restated (mantuoluozk/persistent_lstm_hip): gate order i, f, g, o and the
// c/h recurrence of persistent_lstm_reference.cpp:21-35; fp16 h storage per step and fp32 c of
// persistent_lstm_hip.cu:520-525; the fp32-accumulated head of persistent_lstm_hip.cu:1662-1682.
#include <hip/hip_runtime.h>

#include "plh_internal.h"
#include "../../include/persistent_lstm_hip.h"

namespace plh {
namespace {

typedef f16x8_t f16x8;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
// Wall-clock bound on one hand-off wait (s_memrealtime runs at 100 MHz): 2 s.
constexpr uint64_t kSpinLimitTicks = 200000000ull;
constexpr int kFrag = 64;  // f16x8 elements in one 16 x 32 fragment block (1 KB)

// logistic(x) = 1 / (1 + e^-x), with e^-x = 2^(-x log2 e) on v_exp_f32 and the reciprocal on
// v_rcp_f32.  Saturates cleanly: exp2 -> inf gives 0, exp2 -> 0 gives 1.
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// tanh(x) = 2 logistic(2x) - 1.
__device__ __forceinline__ float tanh_fast(float x) { return fmaf(2.0f, sigmoid_fast(2.0f * x), -1.0f); }

// Barrier that orders LDS traffic only: global stores stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Index (in halfs) of element (row r, k) inside a fragment-ordered [16 x K] block.
__device__ __forceinline__ int frag_index(int r, int k) { return (((k >> 3) << 4) + r) * 8 + (k & 7); }

// Spin (one lane) until *ctr >= need, bounded in wall-clock time, then acquire at agent scope.
// Returns 0 if the wait timed out or any workgroup of the grid has failed.
__device__ int wait_counter(const uint32_t* ctr, uint32_t need, uint32_t* status) {
  uint32_t v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (v < need) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      __builtin_amdgcn_s_sleep(1);
      v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (v >= need) break;
      if (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return 0;
      if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinLimitTicks) {
        __hip_atomic_fetch_or(status, PLH_STATUS_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return 0;
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u ? 1 : 0;
}

// Workgroup -> (layer, tile).  With xcd_map, workgroups are dispatched round-robin over the 8
// XCDs (block b lands on XCD b % 8), and the mapping puts all layers of a tile on one XCD.
__device__ __forceinline__ void block_coords(int b, int ntile, int xcd_map, int& layer, int& tile) {
  if (xcd_map) {
    const int per = ntile >> 3;
    const int r = b >> 3;
    tile = (b & 7) * per + r % per;
    layer = r / per;
  } else {
    layer = b / ntile;
    tile = b % ntile;
  }
}

template <int HP>
struct Tile {
  static constexpr int kWaves = HP / 16;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kKci = HP / 32;  // input-part K chunks (layers >= 1)
  static constexpr int kKcr = HP / 32;  // recurrent K chunks
  static constexpr int kKc = kKci + kKcr;
};

template <int HP, int CH>
__global__ void __launch_bounds__(Tile<HP>::kThreads)
lstm_wavefront_kernel(ForwardArgs a) {
  using C = Tile<HP>;
  constexpr int KCI = C::kKci, KCR = C::kKcr, KC = C::kKc, NT = C::kThreads;
  constexpr int RN = (CH * KCI * kFrag + NT - 1) / NT;  // chunk elements held per thread

  __shared__ f16x8 ring[CH * KCI * kFrag];  // step inputs of the current chunk, fragment order
  __shared__ f16x8 hfrag[2][KCR * kFrag];   // h_{t-1} / h_t, fragment order
  __shared__ int s_ok[2];
  __shared__ int s_tlen;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;   // batch row in the tile: B-operand / D column
  const int kg = lane >> 4;  // K group of the A/B fragments, row group of D
  int layer, tile;
  block_coords(blockIdx.x, a.ntile, a.xcd_map, layer, tile);

  const int grow = a.row0 + tile * 16 + n;
  const bool row_ok = grow < a.row_end;
  int len = 0;
  if (row_ok) {
    len = a.lengths ? a.lengths[grow] : a.T;
    len = len < 0 ? 0 : (len > a.T ? a.T : len);
  }
  if (threadIdx.x == 0) s_tlen = 0;
  __syncthreads();
  if (wave == 0 && kg == 0) atomicMax(&s_tlen, len);
  __syncthreads();
  const int Tt = s_tlen;  // steps this tile runs: the longest row in it

  // Resident weights: A fragments of [W_ih | W_hh] rows for this wave's 16 units, 4 gates.
  f16x8 w[KC][4];
  {
    const f16x8* wp = reinterpret_cast<const f16x8*>(a.wpack) + ((size_t)(layer * C::kWaves + wave) * KC * 4) * kFrag + lane;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int q = 0; q < 4; ++q) w[kc][q] = wp[(kc * 4 + q) * kFrag];
  }
  const int u0 = wave * 16 + kg * 4;  // this lane's 4 hidden units: D rows 4*kg .. 4*kg+3
  f32x4 bias[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) bias[q] = *reinterpret_cast<const f32x4*>(a.bias + ((size_t)layer * 4 + q) * HP + u0);

  // Initial state (nn.LSTM hx) or zeros; h_{-1} goes to hfrag[0].
  float c[4];
  f16x4 hcur;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = u0 + i;
    const bool v = row_ok && u < a.H;
    const size_t si = ((size_t)layer * a.B + grow) * a.H + u;
    c[i] = (v && a.c0) ? (float)a.c0[si] : 0.0f;
    hcur[i] = (v && a.h0) ? a.h0[si] : (_Float16)0.0f;
  }
  const int hoff = frag_index(n, u0);  // where this lane's 4 h values go (8 B, contiguous per wave)
  *reinterpret_cast<f16x4*>(reinterpret_cast<_Float16*>(hfrag[0]) + hoff) = hcur;

  const bool has_up = layer > 0;
  const bool has_down = layer < a.L - 1;
  const int kin = has_up ? KCI : a.kc_in0;  // input fragments per step
  const size_t hstep = (size_t)KCR * kFrag;  // f16x8 per (tile, step) in the hand-off buffer
  const f16x8* in_seq = has_up ? a.hseq + ((size_t)(layer - 1) * a.ntile + tile) * a.T * hstep
                               : a.xp + (size_t)tile * a.T * kin * kFrag;
  _Float16* out_seq_h = has_down ? reinterpret_cast<_Float16*>(a.hseq + ((size_t)layer * a.ntile + tile) * a.T * hstep) + hoff
                                 : nullptr;
  const uint32_t* up_ctr = has_up ? a.counters + (layer - 1) * a.ntile + tile : nullptr;
  uint32_t* my_ctr = a.counters + layer * a.ntile + tile;
  const int sync_tid = C::kWaves > 1 ? 64 : 0;  // the lane that polls upstream (wave 1)

  const int nchunk = (Tt + CH - 1) / CH;
  f16x8 R[RN];
  auto load_chunk = [&](int k) {
    const int s0 = k * CH;
    const int ns = min(CH, Tt - s0);
    const int nel = ns * kin * kFrag;
    const f16x8* src = in_seq + (size_t)s0 * kin * kFrag;
#pragma unroll
    for (int r = 0; r < RN; ++r) {
      const int idx = threadIdx.x + r * NT;
      if (idx < nel) R[r] = src[idx];
    }
  };
  auto store_chunk = [&](int k) {
    const int ns = min(CH, Tt - k * CH);
    const int nel = ns * kin * kFrag;
#pragma unroll
    for (int r = 0; r < RN; ++r) {
      const int idx = threadIdx.x + r * NT;
      if (idx < nel) ring[idx] = R[r];
    }
  };
  auto need_for = [&](int k) -> uint32_t { return (uint32_t)min((k + 1) * CH, Tt); };  // chunk k published

  int wait_idx = 0;
  auto wait_up = [&](uint32_t need) -> bool {  // blocking wait for the upstream layer
    const int slot = wait_idx++ & 1;
    if (threadIdx.x == sync_tid) s_ok[slot] = wait_counter(up_ctr, need, a.status);
    __syncthreads();
    return s_ok[slot] != 0;
  };

  int probe_i = 0;
  int probe_next = a.n_probe > 0 ? a.probe_steps[0] : -1;
  auto write_probe = [&](int p) {
    if (!row_ok) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int u = u0 + i;
      if (u < a.H) {
        const size_t o = (((size_t)p * a.L + layer) * a.B + grow) * a.H + u;
        a.probe_h[o] = (float)hcur[i];
        a.probe_c[o] = c[i];
      }
    }
  };

  bool ok = true;
  uint32_t poll = 0;  // deferred observation of the upstream counter (sync_tid only)
  if (Tt > 0) {
    if (has_up) ok = wait_up(need_for(0));
    if (ok) {
      load_chunk(0);
      store_chunk(0);
    }
    if (ok && nchunk > 1) {
      if (has_up) ok = wait_up(need_for(1));
      if (ok) load_chunk(1);
    }
    if (has_up && threadIdx.x == sync_tid) poll = __hip_atomic_load(up_ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();  // ring (chunk 0) and hfrag[0] visible

  for (int k = 0; ok && k < nchunk; ++k) {
    if (k > 0) {
      // Chunk boundary: publish chunk k-1, move chunk k from VGPRs into the ring, acquire chunk k+1.
      __syncthreads();
      if (has_down && threadIdx.x == 0)
        __hip_atomic_store(my_ctr, (uint32_t)(k * CH), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      store_chunk(k);
      const bool more = k + 1 < nchunk;
      const int slot = wait_idx++ & 1;
      if (has_up && more && threadIdx.x == sync_tid) {
        const uint32_t need = need_for(k + 1);
        int okv;
        if (poll >= need) {
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
          okv = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u ? 1 : 0;
        } else {
          okv = wait_counter(up_ctr, need, a.status);
        }
        poll = __hip_atomic_load(up_ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_ok[slot] = okv;
      }
      __syncthreads();
      if (has_up && more && s_ok[slot] == 0) {
        ok = false;
        break;
      }
      if (more) load_chunk(k + 1);
    }

    const int ns = min(CH, Tt - k * CH);
    for (int s = 0; s < ns; ++s) {
      const int t = k * CH + s;
      f32x4 acc[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = bias[q];
      // Input part (independent of h_{t-1}).
      const f16x8* xr = ring + s * kin * kFrag + lane;
#pragma unroll
      for (int kc = 0; kc < KCI; ++kc) {
        if (kc < kin) {
          const f16x8 xv = xr[kc * kFrag];
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][q], xv, acc[q], 0, 0, 0);
        }
      }
      // Recurrent part.
      const f16x8* hr = &hfrag[t & 1][lane];
#pragma unroll
      for (int kr = 0; kr < KCR; ++kr) {
        const f16x8 hv = hr[kr * kFrag];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[KCI + kr][q], hv, acc[q], 0, 0, 0);
      }

      // Gates and state update on the accumulators: lane holds units u0..u0+3 of row n.
      const bool live = t < len;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ig = sigmoid_fast(acc[0][i]);
        const float fg = sigmoid_fast(acc[1][i]);
        const float gg = tanh_fast(acc[2][i]);
        const float og = sigmoid_fast(acc[3][i]);
        const float cn = fmaf(fg, c[i], ig * gg);
        const _Float16 hn = (_Float16)(og * tanh_fast(cn));
        if (live) {
          c[i] = cn;
          hcur[i] = hn;
        }
      }
      *reinterpret_cast<f16x4*>(reinterpret_cast<_Float16*>(hfrag[(t + 1) & 1]) + hoff) = hcur;
      if (has_down) *reinterpret_cast<f16x4*>(out_seq_h + (size_t)t * hstep * 8) = hcur;
      if (!has_down && a.out_seq && row_ok) {
        _Float16* dst = a.out_seq + ((size_t)grow * a.T + t) * a.H + u0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (u0 + i < a.H) dst[i] = live ? hcur[i] : (_Float16)0.0f;
      }
      if (t + 1 == probe_next) {
        write_probe(probe_i);
        ++probe_i;
        probe_next = probe_i < a.n_probe ? a.probe_steps[probe_i] : -1;
      }
      lds_barrier();
    }
  }

  if (!ok) {
    // A hand-off wait failed (the status word records it and fails every other wait): poison this
    // tile's head outputs and leave.
    if (!has_down && a.out) {
      for (int idx = threadIdx.x; idx < 16 * a.O; idx += NT) {
        const int g = a.row0 + tile * 16 + idx / a.O;
        if (g < a.row_end) a.out[(size_t)g * a.O + idx % a.O] = (_Float16)__builtin_nanf("");
      }
    }
    return;
  }
  if (has_down && Tt > 0) {
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(my_ctr, (uint32_t)Tt, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  }

  // States after the tile's last step (rows that ended earlier were frozen at their last step).
  while (probe_i < a.n_probe) {
    write_probe(probe_i);
    ++probe_i;
  }
  if (row_ok) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int u = u0 + i;
      if (u < a.H) {
        const size_t si = ((size_t)layer * a.B + grow) * a.H + u;
        if (a.h_n) a.h_n[si] = hcur[i];
        if (a.c_n) a.c_n[si] = (_Float16)c[i];
      }
    }
  }

  // Linear head on the final h of the last layer (written to hfrag[Tt & 1] by the last step).
  if (!has_down && a.out) {
    const _Float16* hf = reinterpret_cast<const _Float16*>(hfrag[Tt & 1]);
    for (int idx = threadIdx.x; idx < 16 * a.O; idx += NT) {
      const int r = idx / a.O, o = idx % a.O;
      const int g = a.row0 + tile * 16 + r;
      if (g >= a.row_end) continue;
      const float* wr = a.wlin + (size_t)o * HP;
      float s0 = 0.f, s1 = 0.f;
      for (int k8 = 0; k8 < HP; k8 += 8) {
        const f16x8 hv = *reinterpret_cast<const f16x8*>(hf + frag_index(r, k8));
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          s0 = fmaf((float)hv[j], wr[k8 + j], s0);
          s1 = fmaf((float)hv[j + 1], wr[k8 + j + 1], s1);
        }
      }
      a.out[(size_t)g * a.O + o] = (_Float16)(a.blin[o] + (s0 + s1));
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Weight packing: torch layout -> per-lane MFMA A fragments.
// For 16x16x32 f16, lane l of the A operand holds A[m = l % 16][k = 8 * (l / 16) + j], j < 8.
// Row m of tile (wave w, gate q) is gate column q*H + w*16 + m; K runs over [x | h] in chunks
// of 32: chunks [0, kci) index W_ih columns, [kci, kc) index W_hh columns; out-of-range -> 0.
template <int HP>
__global__ void pack_layer_kernel(const _Float16* __restrict__ w_ih, const _Float16* __restrict__ w_hh, int K,
                                  int H, _Float16* __restrict__ dst) {
  using C = Tile<HP>;
  const size_t total = (size_t)C::kWaves * C::kKc * 4 * 64 * 8;
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int j = e & 7;
  const int lane = (e >> 3) & 63;
  const int q = (e >> 9) & 3;
  const int kc = (int)((e >> 11) % C::kKc);
  const int wv = (int)((e >> 11) / C::kKc);
  const int m = lane & 15, kgrp = lane >> 4;
  const int u = wv * 16 + m;
  const size_t col = (size_t)q * H + u;
  _Float16 v = (_Float16)0.0f;
  if (u < H) {
    if (kc < C::kKci) {
      const int k = kc * 32 + kgrp * 8 + j;
      if (k < K) v = w_ih[col * K + k];
    } else {
      const int k = (kc - C::kKci) * 32 + kgrp * 8 + j;
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

// x [B, T, I] -> xp [ntile][T][kci0][64 lanes] f16x8 in B-fragment order, zero padded.
__global__ void pack_x_kernel(const _Float16* __restrict__ x, int T, int I, int row0, int row_end, int ntile,
                              int kci0, f16x8* __restrict__ xp) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)ntile * T * kci0 * kFrag;
  if (e >= total) return;
  const int lane = (int)(e % kFrag);
  const int kc = (int)((e / kFrag) % kci0);
  const size_t tt = e / ((size_t)kFrag * kci0);
  const int t = (int)(tt % T);
  const int tile = (int)(tt / T);
  const int b = row0 + tile * 16 + (lane & 15);
  const int k0 = kc * 32 + (lane >> 4) * 8;
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

// ---------------------------------------------------------------------------------------------

bool make_geometry(int I, int H, int L, int O, Geometry* g, std::string* why) {
  if (I <= 0 || H <= 0 || L <= 0 || O < 0) {
    *why = "input_size, hidden_size and num_layers must be positive and output_size non-negative";
    return false;
  }
  int HP = 0;
  if (H <= 32) HP = 32;
  else if (H <= 64) HP = 64;
  else if (H <= 128) HP = 128;
  if (HP == 0) {
    *why = "hidden_size > 128 is not implemented by the persistent kernel";
    return false;
  }
  if (I > HP) {
    *why = "input_size larger than the padded hidden size is not implemented";
    return false;
  }
  if (L > 64 || O > 4096) {
    *why = "num_layers > 64 or output_size > 4096 is not implemented";
    return false;
  }
  g->I = I;
  g->H = H;
  g->L = L;
  g->O = O;
  g->HP = HP;
  g->waves = HP / 16;
  g->kci = HP / 32;
  g->kc = 2 * g->kci;
  g->kc_in0 = (I + 31) / 32;
  return true;
}

static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

PackedLayout packed_layout(const Geometry& g) {
  PackedLayout p;
  size_t off = 0;
  p.wpack = off;
  off = align256(off + (size_t)g.L * g.waves * g.kc * 4 * 64 * 8 * sizeof(_Float16));
  p.bias = off;
  off = align256(off + (size_t)g.L * 4 * g.HP * sizeof(float));
  p.wlin = off;
  off = align256(off + (size_t)g.O * g.HP * sizeof(float));
  p.blin = off;
  off = align256(off + (size_t)g.O * sizeof(float));
  p.total = off;
  return p;
}

WorkspaceLayout workspace_layout(const Geometry& g, int seq_len, int chunk_rows) {
  WorkspaceLayout w;
  const size_t ntile = (size_t)chunk_rows / 16;
  const size_t frag_bytes = (size_t)kFrag * 16;  // one 16 x 32 fp16 fragment block
  w.chunk_rows = chunk_rows;
  w.status = 0;
  w.counters = 256;
  w.xp = align256(w.counters + sizeof(uint32_t) * (size_t)g.L * ntile);
  w.hseq = align256(w.xp + ntile * seq_len * g.kc_in0 * frag_bytes);
  w.total = align256(w.hseq + (size_t)(g.L - 1) * ntile * seq_len * g.kci * frag_bytes);
  return w;
}

hipError_t launch_pack_layer(const Geometry& g, int layer, const _Float16* w_ih, const _Float16* w_hh, _Float16* wpack,
                             hipStream_t s) {
  const size_t per_layer = (size_t)g.waves * g.kc * 4 * 64 * 8;
  _Float16* dst = wpack + per_layer * layer;
  const int K = layer == 0 ? g.I : g.H;
  const unsigned grid = blocks_for(per_layer, 256);
  switch (g.HP) {
    case 32: hipLaunchKernelGGL(pack_layer_kernel<32>, grid, 256, 0, s, w_ih, w_hh, K, g.H, dst); break;
    case 64: hipLaunchKernelGGL(pack_layer_kernel<64>, grid, 256, 0, s, w_ih, w_hh, K, g.H, dst); break;
    case 128: hipLaunchKernelGGL(pack_layer_kernel<128>, grid, 256, 0, s, w_ih, w_hh, K, g.H, dst); break;
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

hipError_t launch_pack_x(const Geometry& g, const ForwardArgs& a, hipStream_t s) {
  const size_t n = (size_t)a.ntile * a.T * g.kc_in0 * kFrag;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_x_kernel, blocks_for(n, 256), 256, 0, s, a.x, a.T, a.I, a.row0, a.row_end, a.ntile, g.kc_in0,
                     a.xp);
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

// Steps per hand-off chunk (compile-time tuning knob).
#ifndef PLH_CHUNK_STEPS
#define PLH_CHUNK_STEPS 8
#endif
constexpr int kChunk = PLH_CHUNK_STEPS;

static const void* recurrent_kernel(const Geometry& g) {
  switch (g.HP) {
    case 32: return reinterpret_cast<const void*>(&lstm_wavefront_kernel<32, kChunk>);
    case 64: return reinterpret_cast<const void*>(&lstm_wavefront_kernel<64, kChunk>);
    case 128: return reinterpret_cast<const void*>(&lstm_wavefront_kernel<128, kChunk>);
    default: return nullptr;
  }
}

int recurrent_capacity(const Geometry& g, hipError_t* err) {
  const void* fn = recurrent_kernel(g);
  if (!fn) {
    *err = hipErrorInvalidValue;
    return 0;
  }
  int dev = 0, cus = 0, per_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, g.waves * 64, 0);
  *err = e;
  return e == hipSuccess ? per_cu * cus : 0;
}

hipError_t launch_recurrent(const Geometry& g, const ForwardArgs& a, hipStream_t s) {
  const void* fn = recurrent_kernel(g);
  if (!fn) return hipErrorInvalidValue;
  ForwardArgs args = a;
  void* params[] = {&args};
  return hipLaunchCooperativeKernel(fn, dim3(a.L * a.ntile), dim3(g.waves * 64), params, 0, s);
}

}  // namespace plh
