// plh_kernels.hip -- CDNA4 (gfx950) kernels of the stacked LSTM + Linear inference forward.
//
// Two persistent, weight-stationary, layer-wavefront recurrences (cooperative launches: every
// workgroup of a launch is co-resident and loops over the time steps itself):
//
// lstm_wavefront_kernel (H <= 128): one workgroup per (layer, batch tile of 8 or 16 rows).
//   * each wave owns 16 hidden units and keeps the i, f, g, o rows of [W_ih | W_hh] for them in
//     VGPRs for the whole sequence as fp16 MFMA A fragments (256 KB per layer at H = 128);
//   * per step a wave computes gates^T[64 gate cols, 16 cols] = W[64, K] * [in_t | h_{t-1}]^T with
//     v_mfma_f32_16x16x32_f16 (fp32 accumulate, bias as the initial accumulator); with 8-row tiles
//     the B columns 8..15 repeat rows 0..7 and each lane evaluates two of its four (unit, row)
//     pairs; the next step's input part is issued between this step's gate computations;
//   * the gate nonlinearities and the c/h update run on the accumulator registers; c never leaves
//     VGPRs; h goes to an LDS history ring that also feeds the next step's recurrent MFMAs;
//   * activations live in "fragment order": a [R rows x 32 k] block is stored as [k/8][row][8],
//     i.e. exactly the B operand of one MFMA (lane l reads 16 B at l * 16), in LDS and in the
//     global hand-off buffer, so LDS traffic is conflict-free and global traffic contiguous;
//   * the step input (x for layer 0, h of layer l-1 otherwise) reaches LDS one chunk of CH steps at
//     a time, loaded to VGPRs during the previous chunk, so no step waits on global memory;
//   * the hand-off between layers is a per-(layer, tile) step counter published with an agent-scope
//     release once per chunk and observed with a deferred poll + agent-scope acquire one chunk
//     ahead: layer l+1 works on chunk k while layer l works on later chunks;
//   * the Linear head runs in the last layer's epilogue on the final h held in LDS.
//
// lstm_sliced_kernel (H 129..512): a layer's weights exceed one CU's registers, so S workgroups
// ("slices") share a (layer, 16-row tile) and exchange h every step (see the section below).
//
// Every wait between workgroups is bounded in wall-clock time; a failed wait sets a status bit,
// fails every other wait and poisons the outputs, so the grid always drains.
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

// e^{-k z} as 2^(min(-k z log2 e, 40)) on v_exp_f32.  The cap keeps a product of three (1 + e)
// factors below 2^121 (no overflow) and moves no gate by more than 1e-12 (logistic(-27.7) ~ 1e-12).
constexpr float kExpCap = 40.0f;
__device__ __forceinline__ float exp_neg(float z, float k) {
  return __builtin_amdgcn_exp2f(fminf(z * (-k * kLog2e), kExpCap));
}

// One LSTM cell update (torch gate order i, f, g, o) from the pre-activations and the old c, with
// 5 exponentials and 2 reciprocals instead of the 10 transcendentals of evaluating each of
// sigmoid(i), sigmoid(f), tanh(g), sigmoid(o), tanh(c') as 1 / (1 + e^-x):
//   c' = sigmoid(f) c + sigmoid(i) tanh(g) = [c (1+ei)(1+eg) + (1-eg)(1+ef)] / [(1+ef)(1+ei)(1+eg)]
//   h  = sigmoid(o) tanh(c')               = (1 - ec) / [(1+eo)(1+ec)]
// where ex = e^{-x} for the logistic gates and e^{-2x} for the tanh arguments.  eo alone needs no
// cap: with ec capped, 1 - ec is finite, so eo = +inf gives h = finite * rcp(inf) = 0, the limit.
__device__ __forceinline__ void lstm_cell(float zi, float zf, float zg, float zo, float& c, float& h) {
  const float ei = exp_neg(zi, 1.0f), ef = exp_neg(zf, 1.0f), eg = exp_neg(zg, 2.0f);
  const float eo = __builtin_amdgcn_exp2f(zo * -kLog2e);
  const float a = 1.0f + ei, b = 1.0f + eg, d = 1.0f + ef;
  const float ab = a * b;
  const float cn = fmaf(c, ab, (1.0f - eg) * d) * __builtin_amdgcn_rcpf(d * ab);
  const float ec = exp_neg(cn, 2.0f);
  h = (1.0f - ec) * __builtin_amdgcn_rcpf((1.0f + eo) * (1.0f + ec));
  c = cn;
}

// Barrier that orders LDS traffic only: global stores stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Spin (one lane) until *ctr >= need, bounded by `limit` ticks of s_memrealtime (100 MHz), then
// acquire at agent scope.  Returns 0 if the wait timed out or any workgroup of the grid has failed.
__device__ int wait_counter(const uint32_t* ctr, uint32_t need, uint32_t* status, uint64_t limit) {
  uint32_t v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (v < need) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      __builtin_amdgcn_s_sleep(1);
      v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (v >= need) break;
      if (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return 0;
      if (__builtin_amdgcn_s_memrealtime() - t0 > limit) {
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

template <int HP, int ROWS, int CH>
struct Tile {
  static_assert(ROWS == 8 || ROWS == 16, "tiles hold 8 or 16 batch rows");
  static constexpr int kWaves = HP / 16;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kKci = HP / 32;          // input-part K chunks (layers >= 1)
  static constexpr int kKcr = HP / 32;          // recurrent K chunks
  static constexpr int kKc = kKci + kKcr;
  static constexpr int kFragVec = 4 * ROWS;     // f16x8 per [ROWS x 32] fragment block
  static constexpr int kUpl = ROWS / 4;         // (unit, row) pairs per lane in the epilogue
  // f16x8 elements each thread moves per chunk (input ring fill, hand-off copy)
  static constexpr int kRn = (CH * kKci * kFragVec + kThreads - 1) / kThreads;
};

// Offset (in halfs) of element (row r, k) in a fragment-ordered [ROWS x K] block: the block of K
// chunk k/32 is stored as [k/8 % 4][row][8], i.e. exactly the B operand of one MFMA.
template <int ROWS>
__device__ __forceinline__ int frag_index(int r, int k) { return ((k >> 3) * ROWS + r) * 8 + (k & 7); }

// a if !sel else b, as one v_cndmask: the empty asm hides that a and b are elements of one vector,
// which would otherwise be turned into a dynamically indexed extract (three compares and selects).
__device__ __forceinline__ float pick(bool sel, float a, float b) {
  asm volatile("" : "+v"(b));
  return sel ? b : a;
}

// The persistent layer-wavefront recurrence.  Template: padded hidden size HP, batch rows per
// workgroup ROWS (16, or 8 with the MFMA's B columns 8..15 duplicating rows 0..7 so each lane
// evaluates two (unit, row) pairs instead of four), steps per hand-off chunk CH, and RAGGED: rows
// may end before the tile's last step (lengths given); without it every row is live at every step
// and the state-freezing selects are compiled out.
template <int HP, int ROWS, int CH, bool RAGGED>
__global__ void __launch_bounds__(HP / 16 * 64)
lstm_wavefront_kernel(ForwardArgs a) {
  using C = Tile<HP, ROWS, CH>;
  constexpr int KCI = C::kKci, KCR = C::kKcr, KC = C::kKc, NT = C::kThreads, FV = C::kFragVec;
  constexpr int UPL = C::kUpl, RN = C::kRn;

  __shared__ f16x8 ring[CH * KCI * FV];   // step inputs of the current chunk
  __shared__ f16x8 hist[CH * KCR * FV];   // h of the chunk's steps; slot (t-1) % CH feeds step t
  __shared__ int s_ok[2];
  __shared__ int s_tlen;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;            // B-operand / D column
  const int kg = lane >> 4;           // K group of the A/B fragments, row group of D
  const int r = n & (ROWS - 1);       // batch row in the tile
  const int fl = kg * ROWS + r;       // this lane's B fragment within a block
  int layer, tile;
  block_coords(blockIdx.x, a.ntile, a.xcd_map, layer, tile);

  const int grow = a.row0 + tile * ROWS + r;
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
    const f16x8* wp = reinterpret_cast<const f16x8*>(a.wpack) + ((size_t)(layer * C::kWaves + wave) * KC * 4) * 64 + lane;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int q = 0; q < 4; ++q) w[kc][q] = wp[(kc * 4 + q) * 64];
  }
  // D rows of this lane: units u0 .. u0+3 of row n; it evaluates UPL of them, starting at uo.
  const int u0 = wave * 16 + kg * 4;
  const int ibase = (ROWS == 8 && n >= 8) ? 2 : 0;
  const int uo = u0 + ibase;
  f32x4 bias[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) bias[q] = *reinterpret_cast<const f32x4*>(a.bias + ((size_t)layer * 4 + q) * HP + u0);

  // Initial state (nn.LSTM hx) or zeros; h_{-1} goes to history slot CH-1.
  typedef _Float16 hvec __attribute__((ext_vector_type(UPL)));
  float c[UPL];
  hvec hcur;
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = uo + j;
    const bool v = row_ok && u < a.H;
    const size_t si = ((size_t)layer * a.B + grow) * a.H + u;
    c[j] = (v && a.c0) ? (float)a.c0[si] : 0.0f;
    hcur[j] = (v && a.h0) ? a.h0[si] : (_Float16)0.0f;
  }
  const int hoff = frag_index<ROWS>(r, uo);  // where this lane's UPL h values go (contiguous)
  auto hist_h = [&](int slot) -> _Float16* { return reinterpret_cast<_Float16*>(hist + slot * (KCR * FV)) + hoff; };
  *reinterpret_cast<hvec*>(hist_h(CH - 1)) = hcur;

  const bool has_up = layer > 0;
  const bool has_down = layer < a.L - 1;
  const int kin = has_up ? KCI : a.kc_in0;  // input fragment blocks per step
  const size_t hstep = (size_t)KCR * FV;     // f16x8 per (tile, step) in the hand-off buffer
  const f16x8* in_seq = has_up ? a.hseq + ((size_t)(layer - 1) * a.ntile + tile) * a.T * hstep
                               : a.xp + (size_t)tile * a.T * kin * FV;
  f16x8* out_seq_h = has_down ? a.hseq + ((size_t)layer * a.ntile + tile) * a.T * hstep : nullptr;
  const uint32_t* up_ctr = has_up ? a.counters + (layer - 1) * a.ntile + tile : nullptr;
  uint32_t* my_ctr = a.counters + layer * a.ntile + tile;
  const int sync_tid = C::kWaves > 1 ? 64 : 0;  // the lane that polls upstream (wave 1)

  const int nchunk = (Tt + CH - 1) / CH;
  f16x8 R[RN];
  auto load_chunk = [&](int k) {
    const int s0 = k * CH;
    const int nel = min(CH, Tt - s0) * kin * FV;
    const f16x8* src = in_seq + (size_t)s0 * kin * FV;
#pragma unroll
    for (int i = 0; i < RN; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (idx < nel) R[i] = src[idx];
    }
  };
  // The ring always holds KCI fragment blocks per step; layer 0 fills the first kin of them (the
  // others stay zero from the initialisation), so every layer runs the same branch-free MFMAs.
  auto store_chunk = [&](int k) {
    const int per = kin * FV;
    const int nel = min(CH, Tt - k * CH) * per;
#pragma unroll
    for (int i = 0; i < RN; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (idx < nel) ring[(idx / per) * (KCI * FV) + idx % per] = R[i];
    }
  };
  // Hand-off copy of chunk k's h history (LDS) to the global sequence buffer.
  auto copy_out = [&](int k) {
    const int nel = min(CH, Tt - k * CH) * (KCR * FV);
    f16x8* dst = out_seq_h + (size_t)k * CH * hstep;
#pragma unroll
    for (int i = 0; i < RN; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (idx < nel) dst[idx] = hist[idx];
    }
  };
  auto need_for = [&](int k) -> uint32_t { return (uint32_t)min((k + 1) * CH, Tt); };  // chunk k published

  int wait_idx = 0;
  auto wait_up = [&](uint32_t need) -> bool {  // blocking wait for the upstream layer
    const int slot = wait_idx++ & 1;
    if (threadIdx.x == sync_tid) s_ok[slot] = wait_counter(up_ctr, need, a.status, a.wait_ticks);
    __syncthreads();
    return s_ok[slot] != 0;
  };

  int probe_i = 0;
  int probe_next = a.n_probe > 0 ? a.probe_steps[0] : -1;
  auto write_probe = [&](int p) {
    if (!row_ok) return;
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
      const int u = uo + j;
      if (u < a.H) {
        const size_t o = (((size_t)p * a.L + layer) * a.B + grow) * a.H + u;
        a.probe_h[o] = (float)hcur[j];
        a.probe_c[o] = c[j];
      }
    }
  };

  for (int i = threadIdx.x; i < CH * KCI * FV; i += NT) ring[i] = f16x8{};
  __syncthreads();

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
  __syncthreads();  // ring (chunk 0) and the initial h visible

  const bool hi = ibase != 0;
  for (int k = 0; ok && k < nchunk; ++k) {
    if (k > 0) {
      // Chunk boundary: hand chunk k-1's h to global memory, move chunk k's input from VGPRs into
      // the ring, acquire chunk k+1 of the upstream layer and start loading it.
      __syncthreads();
      if (has_down) copy_out(k - 1);
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
          okv = wait_counter(up_ctr, need, a.status, a.wait_ticks);
        }
        poll = __hip_atomic_load(up_ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_ok[slot] = okv;
      }
      __syncthreads();  // also orders every wave's hand-off stores before the publication below
      if (has_up && more && s_ok[slot] == 0) {
        ok = false;
        break;
      }
      if (more) load_chunk(k + 1);
    }

    const int ns = min(CH, Tt - k * CH);
    // Chunk k-1 is published halfway through chunk k: its stores have drained by then, so the
    // release costs the publishing wave little.
    const int pub_s = (k > 0 && has_down) ? min(CH / 2, ns - 1) : -1;
    f32x4 acc_next[4];
    {
      const f16x8* xr = ring + fl;
      f16x8 xv[KCI];
#pragma unroll
      for (int kc = 0; kc < KCI; ++kc) xv[kc] = xr[kc * FV];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc_next[q] = bias[q];
#pragma unroll
      for (int kc = 0; kc < KCI; ++kc)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc_next[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][q], xv[kc], acc_next[q], 0, 0, 0);
    }
    for (int s = 0; s < ns; ++s) {
      const int t = k * CH + s;
      f32x4 acc[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = acc_next[q];
      // Recurrent part: h_{t-1} from the history slot of the previous step.
      const f16x8* hr = hist + (s == 0 ? CH - 1 : s - 1) * (KCR * FV) + fl;
      f16x8 hv[KCR];
#pragma unroll
      for (int kr = 0; kr < KCR; ++kr) hv[kr] = hr[kr * FV];
#pragma unroll
      for (int kr = 0; kr < KCR; ++kr)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[KCI + kr][q], hv[kr], acc[q], 0, 0, 0);

      // Next step's input part (the chunk's last step recomputes a discarded in-range step),
      // interleaved with this step's gate math: each (unit, row) piece of the epilogue is preceded
      // by its share of the next step's MFMAs and fenced with sched_barrier, so the matrix core
      // runs while the VALU evaluates the gates (in-order issue would otherwise queue all VALU
      // work behind the MFMAs).
      const f16x8* xr = ring + min(s + 1, ns - 1) * (KCI * FV) + fl;
      f16x8 xv[KCI];
#pragma unroll
      for (int kc = 0; kc < KCI; ++kc) xv[kc] = xr[kc * FV];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc_next[q] = bias[q];
      const bool live = t < len;
      constexpr int kMfmaPerPiece = (KCI * 4 + UPL - 1) / UPL;
#pragma unroll
      for (int j = 0; j < UPL; ++j) {
#pragma unroll
        for (int m = j * kMfmaPerPiece; m < (j + 1) * kMfmaPerPiece && m < KCI * 4; ++m) {
          const int kc = m / 4, q = m % 4;
          acc_next[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][q], xv[kc], acc_next[q], 0, 0, 0);
        }
        // this lane's pair j: D element ibase + j of every gate tile (one v_cndmask each)
        float z[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) z[q] = pick(hi, acc[q][j], acc[q][2 + j % 2]);
        float cn = c[j], hn;
        lstm_cell(z[0], z[1], z[2], z[3], cn, hn);
        if constexpr (RAGGED) {
          // selects, not a branch: rows past their length keep their state
          c[j] = live ? cn : c[j];
          hcur[j] = live ? (_Float16)hn : hcur[j];
        } else {
          c[j] = cn;
          hcur[j] = (_Float16)hn;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      *reinterpret_cast<hvec*>(hist_h(s)) = hcur;
      if (!has_down && a.out_seq && row_ok) {
        _Float16* dst = a.out_seq + ((size_t)grow * a.T + t) * a.H + uo;
#pragma unroll
        for (int j = 0; j < UPL; ++j)
          if (uo + j < a.H) dst[j] = live ? hcur[j] : (_Float16)0.0f;
      }
      if (t + 1 == probe_next) {
        write_probe(probe_i);
        ++probe_i;
        probe_next = probe_i < a.n_probe ? a.probe_steps[probe_i] : -1;
      }
      if (s == pub_s && threadIdx.x == 0)
        __hip_atomic_store(my_ctr, (uint32_t)(k * CH), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      lds_barrier();
    }
  }

  if (!ok) {
    // A hand-off wait failed (the status word records it and fails every other wait): poison this
    // tile's head outputs and leave.
    if (!has_down && a.out) {
      for (int idx = threadIdx.x; idx < ROWS * a.O; idx += NT) {
        const int g = a.row0 + tile * ROWS + idx / a.O;
        if (g < a.row_end) a.out[(size_t)g * a.O + idx % a.O] = (_Float16)__builtin_nanf("");
      }
    }
    return;
  }
  if (has_down && Tt > 0) {
    __syncthreads();
    copy_out(nchunk - 1);
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(my_ctr, (uint32_t)Tt, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Steps past the tile's longest row were never visited: their output sequence is zero.
  if (!has_down && a.out_seq && row_ok) {
    for (int t = Tt; t < a.T; ++t) {
      _Float16* dst = a.out_seq + ((size_t)grow * a.T + t) * a.H + uo;
#pragma unroll
      for (int j = 0; j < UPL; ++j)
        if (uo + j < a.H) dst[j] = (_Float16)0.0f;
    }
  }

  // States after the tile's last step (rows that ended earlier were frozen at their last step).
  while (probe_i < a.n_probe) {
    write_probe(probe_i);
    ++probe_i;
  }
  if (row_ok) {
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
      const int u = uo + j;
      if (u < a.H) {
        const size_t si = ((size_t)layer * a.B + grow) * a.H + u;
        if (a.h_n) a.h_n[si] = hcur[j];
        if (a.c_n) a.c_n[si] = (_Float16)c[j];
      }
    }
  }

  // Linear head on the final h of the last layer (history slot of the tile's last step).
  if (!has_down && a.out) {
    const _Float16* hf = reinterpret_cast<const _Float16*>(hist + ((Tt + CH - 1) % CH) * (KCR * FV));
    for (int idx = threadIdx.x; idx < ROWS * a.O; idx += NT) {
      const int rr = idx / a.O, o = idx % a.O;
      const int g = a.row0 + tile * ROWS + rr;
      if (g >= a.row_end) continue;
      const float* wr = a.wlin + (size_t)o * HP;
      float s0 = 0.f, s1 = 0.f;
      for (int k8 = 0; k8 < HP; k8 += 8) {
        const f16x8 hv = *reinterpret_cast<const f16x8*>(hf + frag_index<ROWS>(rr, k8));
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
// Hidden sizes above 128.  A layer's [W_ih | W_hh] (1 MB at H = 256, 4 MB at H = 512) no longer fits
// one CU's register file, so each (layer, 16-row tile) is served by S workgroups ("slices"), each
// keeping the gate rows of HS = HP / S hidden units resident in VGPRs:
//   * the 8 waves of a slice form HS/16 unit groups; within a group, KSP waves hold the input part
//     (W_ih columns, 256 per wave) and KSP waves the recurrent part (W_hh columns), so every wave's
//     resident weights are 8 K-chunks x 4 gates = 128 VGPRs;
//   * per step each wave computes its partial gate sums with MFMA, the partials meet in LDS, and
//     the group's waves split the gate math of its 16 units x 16 rows (two units per lane);
//   * the slices exchange h_t every step through a small ring of tagged words (below); the next
//     layer still receives h through the hand-off buffer and a per-(layer, tile) step counter
//     published once per chunk, so layers run as a wavefront.
//
// Tagged exchange.  One step's h of a tile is HP x 16 halfs, stored as 64-bit words
// {h[u], h[u+1], tag = t + 1} in writer order ([slice][wave][lane], one word per active lane), so
// each wave's stores and each reader's loads cover contiguous 512-byte runs; the reader scatters
// the payloads into B-fragment order in LDS.  A reader spins on
// the words themselves until every tag it needs equals t + 1: no store-completion wait, barrier or
// counter round trip sits between a slice's epilogue and its siblings' next step.  Every word is
// written and read with agent-scope relaxed 64-bit atomics (sc1), which are single-copy atomic and
// coherent across the XCDs' L2 caches without cache maintenance.  Two ring slots suffice: a slice
// can overwrite slot t % 2 with h_{t+2} only after it has read h_{t+1} of every sibling, and a
// sibling writes h_{t+1} only after it has read h_t from every slice.  The ring is zeroed before
// each launch (tags start at 1).
//
// Hand-off to the next layer: h is also stored to the hand-off buffer with agent-scope relaxed
// stores; at the end of each chunk every thread waits for its stores to complete (s_waitcnt)
// before the barrier that precedes a relaxed counter increment.  The next layer reads the buffer
// with ordinary loads after an agent-scope acquire, which invalidates any stale copy in its L2.
template <int HP>
struct Sliced {
  static constexpr int kKsp = HP / 256;     // waves per K part of a unit group
  static constexpr int kGroups = 4 / kKsp;  // 16-unit groups per workgroup
  static constexpr int kHs = 16 * kGroups;  // hidden units per workgroup
  static constexpr int kS = HP / kHs;       // workgroups per (layer, tile)
  static constexpr int kKch = HP / 32;      // K chunks of one part
  static constexpr int kWpg = 2 * kKsp;     // waves per unit group
  static constexpr int kWords = HP * 8;     // tagged words of one step's h of a 16-row tile
  // Wave roles: waves 0..3 hold W_ih parts, waves 4..7 W_hh parts, so each SIMD (wave w % 4) runs one
  // of each and the input waves' MFMAs for step t+1 overlap the recurrent critical path of step t.
  // Wave w serves unit group (w % 4) / KSP as member e = (w / 4) * KSP + w % KSP of the group
  // (e < KSP: input part, quarter e; else recurrent part, quarter e - KSP).
  static __host__ __device__ constexpr int group_of(int w) { return (w & 3) / kKsp; }
  static __host__ __device__ constexpr int member_of(int w) { return (w >> 2) * kKsp + (w & (kKsp - 1)); }
  static __host__ __device__ constexpr int wave_of(int g, int e) { return (e / kKsp) * 4 + g * kKsp + e % kKsp; }
};

__device__ __forceinline__ uint64_t tag_word(_Float16 a, _Float16 b, uint32_t tag) {
  union { _Float16 h[2]; uint32_t u; } v;
  v.h[0] = a;
  v.h[1] = b;
  return (uint64_t)v.u | ((uint64_t)tag << 32);
}

__device__ __forceinline__ uint32_t word_tag(uint64_t w) { return (uint32_t)(w >> 32); }

__device__ __forceinline__ uint64_t load_agent_u64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup -> (layer, tile, slice).  With xcd_map the S slices of a (layer, tile) share an XCD.
__device__ __forceinline__ void sliced_coords(int b, int ntile, int S, int xcd_map, int& layer, int& tile,
                                              int& slice) {
  int grp;
  if (xcd_map) {
    const int j = b >> 3;
    slice = j % S;
    grp = (j / S) * 8 + (b & 7);
  } else {
    slice = b % S;
    grp = b / S;
  }
  layer = grp / ntile;
  tile = grp % ntile;
}

// NTI 16-row tiles per workgroup.  With NTI = 2 the two tiles are software-pipelined: a tile's
// gather of h_t (issued right after its own words were stored) is completed in the middle of the
// other tile's step, after that tile's gate math and before its stores, so the exchange latency
// hides behind the other tile's work and the wait for the gather's loads (one in-order counter
// covers loads and stores) finds only operations issued a whole phase earlier.
// The layer hand-off is published every PUB chunks: the publication waits for every outstanding
// memory operation of the workgroup (stores and gather loads share one counter), so publishing
// less often keeps that wait off most steps.
template <int HP, int CH, int NTI>
__global__ void __launch_bounds__(512) lstm_sliced_kernel(ForwardArgs a) {
  using C = Sliced<HP>;
  constexpr int KSP = C::kKsp, HS = C::kHs, S = C::kS, KCH = C::kKch, WPG = C::kWpg;
  constexpr int NT = 512, FV = 64;                  // 16-row fragment blocks
  constexpr int RN = (CH * KCH * FV + NT - 1) / NT;  // f16x8 of a chunk's input each thread moves
  constexpr int KCW = 8;                            // K chunks per wave
  constexpr int PUB = NTI == 1 ? 1 : 4;             // chunks per hand-off publication
  static_assert(KCH * FV % NT == 0, "whole fragments per thread");
  static_assert(NTI == 1 || NTI == 2, "one or two tiles per workgroup");

  __shared__ f16x8 ring[NTI][CH * KCH * FV];  // step inputs of the current chunk (all HP input units)
  __shared__ f16x8 hbuf[NTI][KCH * FV];       // h_{t-1} of all HP units
  // Partial gate sums of every wave: per tile with two tiles (the other tile's gather barrier
  // separates a tile's epilogue from the next writes), double-buffered by step with one.
  __shared__ f32x4 part[2][8][4][64];
  __shared__ float2 s_bias[4][HS / 2];  // b_ih + b_hh of this slice's units, by gate and unit pair
  __shared__ int s_ok[2];
  __shared__ int s_fail;
  __shared__ int s_tlen;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int layer, tgrp, slice;
  sliced_coords(blockIdx.x, a.ntile / NTI, S, a.xcd_map, layer, tgrp, slice);
  const int g = C::group_of(wave), ew = C::member_of(wave);
  const bool recurrent = ew >= KSP;  // this wave holds W_hh columns
  const int kq = ew % KSP;           // which 256-column quarter of its part

  // Epilogue mapping: each active lane evaluates units eu, eu + 1 of row en.  The partial sums of
  // (unit 4 kgx + i, row en) sit in element i of lane 16 kgx + en of every wave of the group.
  const int en = lane & 15;
  const int kgx = WPG == 2 ? (lane >> 4) : ew;
  const int pp = WPG == 2 ? ew : ((lane >> 4) & 1);
  const bool active = WPG == 2 || lane < 32;
  const int pl = kgx * 16 + en;
  const int eu = slice * HS + g * 16 + kgx * 4 + 2 * pp;

  int grow[NTI], len[NTI];
  bool row_ok[NTI];
  if (threadIdx.x == 0) {
    s_tlen = 0;
    s_fail = 0;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NTI; ++i) {
    grow[i] = a.row0 + (tgrp * NTI + i) * 16 + en;
    row_ok[i] = grow[i] < a.row_end;
    len[i] = 0;
    if (row_ok[i]) {
      len[i] = a.lengths ? a.lengths[grow[i]] : a.T;
      len[i] = len[i] < 0 ? 0 : (len[i] > a.T ? a.T : len[i]);
    }
    if (wave == 0 && lane < 16) atomicMax(&s_tlen, len[i]);
  }
  __syncthreads();
  const int Tt = s_tlen;  // steps of this workgroup: the longest row of its tiles

  f16x8 w[KCW][4];
  {
    const f16x8* wp = reinterpret_cast<const f16x8*>(a.wpack) +
                      ((size_t)((layer * S + slice) * 8 + wave) * KCW * 4) * 64 + lane;
#pragma unroll
    for (int kc = 0; kc < KCW; ++kc)
#pragma unroll
      for (int q = 0; q < 4; ++q) w[kc][q] = wp[(kc * 4 + q) * 64];
  }
  for (int idx = threadIdx.x; idx < 4 * HS / 2; idx += NT) {
    const int q = idx / (HS / 2), up = idx % (HS / 2);
    const float* b = a.bias + ((size_t)layer * 4 + q) * HP + slice * HS + 2 * up;
    s_bias[q][up] = float2{b[0], b[1]};
  }

  float c[NTI][2];
  _Float16 hcur[NTI][2];
#pragma unroll
  for (int i = 0; i < NTI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int u = eu + j;
      const bool v = row_ok[i] && u < a.H;
      const size_t si = ((size_t)layer * a.B + grow[i]) * a.H + u;
      c[i][j] = (v && a.c0) ? (float)a.c0[si] : 0.0f;
      hcur[i][j] = (v && a.h0) ? a.h0[si] : (_Float16)0.0f;
    }
  // h_{-1} of all units into hbuf (fragment order)
  for (int idx = threadIdx.x; idx < NTI * KCH * FV; idx += NT) {
    const int i = idx / (KCH * FV), kc = idx / FV % KCH, l = idx % FV;
    const int gr = a.row0 + (tgrp * NTI + i) * 16 + (l & 15);
    const int k0 = kc * 32 + (l >> 4) * 8;
    f16x8 v = {};
    if (a.h0 && gr < a.row_end) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (k0 + j < a.H) v[j] = a.h0[((size_t)layer * a.B + gr) * a.H + k0 + j];
    }
    hbuf[i][idx % (KCH * FV)] = v;
  }

  const bool has_up = layer > 0;
  const bool has_down = layer + 1 < a.L;
  const int kin = has_up ? KCH : a.kc_in0;
  const size_t hstep = (size_t)KCH * FV;
  const int tile0 = tgrp * NTI;  // first 16-row tile of this workgroup
  auto in_seq = [&](int i) -> const f16x8* {
    return has_up ? a.hseq + ((size_t)(layer - 1) * a.ntile + tile0 + i) * a.T * hstep
                  : a.xp + (size_t)(tile0 + i) * a.T * kin * FV;
  };
  auto my_seq = [&](int i) -> f16x8* { return a.hseq + ((size_t)layer * a.ntile + tile0 + i) * a.T * hstep; };
  auto xr = [&](int i) -> uint64_t* { return a.xring + ((size_t)layer * a.ntile + tile0 + i) * 2 * C::kWords; };
  const int hoff = ((eu >> 3) * 16 + en) * 8 + (eu & 7);  // halfs: (row en, unit eu) in a step block
  constexpr int WL = WPG == 2 ? 64 : 32;  // tagged words each wave writes per step (its active lanes)
  constexpr int NW = C::kWords / NT;       // tagged words each thread gathers per step
  static_assert(S * 8 * WL == C::kWords && C::kWords % NT == 0, "writer-order ring covers one step");
  const int woff = (slice * 8 + wave) * WL + (lane & (WL - 1));  // this lane's word in a ring slot
  // LDS destination (u32 index into hbuf) of the r-th word this thread gathers.
  auto gdst = [&](int r) -> int {
    const int wd = threadIdx.x + r * NT;
    const int sl = wd / (8 * WL), wv_ = (wd / WL) % 8, ln = wd % WL;
    const int g_ = C::group_of(wv_), ew_ = C::member_of(wv_);
    const int kgx_ = WPG == 2 ? (ln >> 4) : ew_;
    const int pp_ = WPG == 2 ? ew_ : ((ln >> 4) & 1);
    const int eu_ = sl * HS + g_ * 16 + kgx_ * 4 + 2 * pp_;
    return ((eu_ >> 3) * 16 + (ln & 15)) * 4 + ((eu_ & 7) >> 1);
  };
  auto up_ctr = [&](int i) -> const uint32_t* { return a.counters + (layer - 1) * a.ntile + tile0 + i; };
  auto my_ctr = [&](int i) -> uint32_t* { return a.counters + layer * a.ntile + tile0 + i; };
  const int sync_tid = 64;

  const int nchunk = (Tt + CH - 1) / CH;
  f16x8 R[NTI][RN];
  auto load_chunk = [&](int k) {
    const int s0 = k * CH;
    const int nel = min(CH, Tt - s0) * kin * FV;
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      const f16x8* src = in_seq(i) + (size_t)s0 * kin * FV;
#pragma unroll
      for (int r = 0; r < RN; ++r) {
        const int idx = threadIdx.x + r * NT;
        if (idx < nel) R[i][r] = src[idx];
      }
    }
  };
  auto store_chunk = [&](int k) {
    const int per = kin * FV;
    const int nel = min(CH, Tt - k * CH) * per;
#pragma unroll
    for (int i = 0; i < NTI; ++i)
#pragma unroll
      for (int r = 0; r < RN; ++r) {
        const int idx = threadIdx.x + r * NT;
        if (idx < nel) ring[i][(idx / per) * (KCH * FV) + idx % per] = R[i][r];
      }
  };
  // Slice-steps of the upstream tile published once its chunk k is complete (publications cover
  // PUB chunks, or the whole sequence at its end).
  auto need_up = [&](int k) -> uint32_t {
    const int steps = ((k + PUB) / PUB) * PUB * CH;
    return (uint32_t)(S * min(steps, Tt));
  };

  int wait_idx = 0;
  // Acquire chunk k of every tile of the upstream layer.  `poll` holds the last counter value the
  // polling lane saw, per tile, so a chunk that was already published costs only the acquire fence.
  uint32_t poll[NTI];
#pragma unroll
  for (int i = 0; i < NTI; ++i) poll[i] = 0;
  auto acquire_up = [&](int k) -> bool {
    const int slot = wait_idx++ & 1;
    if (threadIdx.x == sync_tid) {
      const uint32_t need = need_up(k);
      int okv = 1;
#pragma unroll
      for (int i = 0; i < NTI; ++i) {
        if (!okv) break;
        if (poll[i] >= need) {
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
          okv = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u ? 1 : 0;
        } else {
          okv = wait_counter(up_ctr(i), need, a.status, a.wait_ticks);
        }
        poll[i] = __hip_atomic_load(up_ctr(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      s_ok[slot] = okv;
    }
    __syncthreads();
    return s_ok[slot] != 0;
  };

  auto pslot = [&](int i, int t) -> int { return NTI == 2 ? i : (t & 1); };
  // This wave's partial gate sums of tile i for step t: its K part of [ring slot s | h_{t-1}].
  auto partials = [&](int i, int t, int s) {
    const f16x8* src = (recurrent ? hbuf[i] : ring[i] + s * (KCH * FV)) + kq * KCW * FV + lane;
    f32x4 acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < KCW; ++kc) {
      const f16x8 bv = src[kc * FV];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][q], bv, acc[q], 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) part[pslot(i, t)][wave][q][lane] = acc[q];
  };

  // Gather words of tile i, step t: issued right after the tile's own words are stored.
  uint64_t wv[NTI][NW];
  auto issue_gather = [&](int i, int t) {
    const uint64_t* src = xr(i) + (size_t)(t & 1) * C::kWords + threadIdx.x;
#pragma unroll
    for (int r = 0; r < NW; ++r) wv[i][r] = load_agent_u64(src + r * NT);
  };
  // Complete the gather of tile i, step t, into hbuf[i]: re-poll the words whose tag is not t + 1
  // yet.  Before spinning, the input waves compute tile i's partials for step t + 1 (ring slot
  // s_next; -1: none).  False (uniformly) if any wait of the workgroup failed.
  auto complete_gather = [&](int i, int t, int s_next) -> bool {
    if (!recurrent && s_next >= 0) partials(i, t + 1, s_next);
    const uint64_t* src = xr(i) + (size_t)(t & 1) * C::kWords + threadIdx.x;
    const uint32_t want = (uint32_t)t + 1u;
    uint64_t t0 = 0;
    for (int spin = 0;; ++spin) {
      bool ready = true;
#pragma unroll
      for (int r = 0; r < NW; ++r) ready = ready && word_tag(wv[i][r]) == want;
      if (ready) break;
      if (spin == 0) {
        t0 = __builtin_amdgcn_s_memrealtime();
      } else if ((spin & 15) == 0) {
        if (__hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
          s_fail = 1;
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t0 > a.wait_ticks) {
          __hip_atomic_fetch_or(a.status, PLH_STATUS_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          s_fail = 1;
          break;
        }
      }
#pragma unroll
      for (int r = 0; r < NW; ++r)
        if (word_tag(wv[i][r]) != want) wv[i][r] = load_agent_u64(src + r * NT);
    }
    uint32_t* hb32 = reinterpret_cast<uint32_t*>(hbuf[i]);
#pragma unroll
    for (int r = 0; r < NW; ++r) hb32[gdst(r)] = (uint32_t)wv[i][r];
    lds_barrier();
    return s_fail == 0;
  };

  // Gate math of tile i, step t, from the group's partial sums plus the bias.
  auto gate_math = [&](int i, int t) {
    const bool live = t < len[i];
    if (!active) return;
    float z[4][2];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float2 bv = s_bias[q][(eu - slice * HS) >> 1];
      z[q][0] = bv.x;
      z[q][1] = bv.y;
#pragma unroll
      for (int e = 0; e < WPG; ++e) {
        const float2 v = reinterpret_cast<const float2*>(&part[pslot(i, t)][C::wave_of(g, e)][q][pl])[pp];
        z[q][0] += v.x;
        z[q][1] += v.y;
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float cn = c[i][j], hn;
      lstm_cell(z[0][j], z[1][j], z[2][j], z[3][j], cn, hn);
      c[i][j] = live ? cn : c[i][j];
      hcur[i][j] = live ? (_Float16)hn : hcur[i][j];
    }
  };
  // Stores of tile i, step t: the tagged words, the hand-off and the output sequence.
  auto store_h = [&](int i, int t) {
    if (!active) return;
    const bool live = t < len[i];
    __hip_atomic_store(xr(i) + (size_t)(t & 1) * C::kWords + woff, tag_word(hcur[i][0], hcur[i][1], (uint32_t)t + 1u),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (has_down) {
      union { _Float16 h[2]; uint32_t u; } v;
      v.h[0] = hcur[i][0];
      v.h[1] = hcur[i][1];
      __hip_atomic_store(reinterpret_cast<uint32_t*>(reinterpret_cast<_Float16*>(my_seq(i) + (size_t)t * hstep) + hoff),
                         v.u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!has_down && a.out_seq && row_ok[i]) {
      _Float16* dst = a.out_seq + ((size_t)grow[i] * a.T + t) * a.H + eu;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (eu + j < a.H) dst[j] = live ? hcur[i][j] : (_Float16)0.0f;
    }
  };

  int probe_i = 0;
  int probe_next = a.n_probe > 0 ? a.probe_steps[0] : -1;
  auto write_probe = [&](int pi) {
    if (!active) return;
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      if (!row_ok[i]) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int u = eu + j;
        if (u < a.H) {
          const size_t o = (((size_t)pi * a.L + layer) * a.B + grow[i]) * a.H + u;
          a.probe_h[o] = (float)hcur[i][j];
          a.probe_c[o] = c[i][j];
        }
      }
    }
  };
  // Hand-off stores complete, then count `steps` more steps of every tile of this workgroup.
  auto publish = [&](uint32_t steps) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < NTI) __hip_atomic_fetch_add(my_ctr(threadIdx.x), steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };

  for (int idx = threadIdx.x; idx < NTI * CH * KCH * FV; idx += NT) ring[idx / (CH * KCH * FV)][idx % (CH * KCH * FV)] = f16x8{};
  __syncthreads();

  bool ok = true;
  if (Tt > 0) {
    if (has_up) ok = acquire_up(0);
    if (ok) {
      load_chunk(0);
      store_chunk(0);
    }
    if (ok && nchunk > 1) {
      if (has_up) ok = acquire_up(1);
      if (ok) load_chunk(1);
    }
  }
  __syncthreads();

  uint32_t unpublished = 0;  // steps computed since the last publication
  for (int k = 0; ok && k < nchunk; ++k) {
    if (k > 0) {
      if (has_down && k % PUB == 0) {
        publish(unpublished);
        unpublished = 0;
      } else {
        __syncthreads();
      }
      store_chunk(k);
      const bool more = k + 1 < nchunk;
      if (has_up && more) {
        if (!acquire_up(k + 1)) {
          ok = false;
          break;
        }
      } else {
        __syncthreads();
      }
      if (more) load_chunk(k + 1);
    }
    const int ns = min(CH, Tt - k * CH);
    for (int s = 0; s < ns && ok; ++s) {
      const int t = k * CH + s;
      if constexpr (NTI == 1) {
        // h_{t-1} (the input partials for step t are computed while the words arrive).
        if (t > 0 && !complete_gather(0, t - 1, s)) {
          ok = false;
          break;
        }
        if (t == 0 || recurrent) partials(0, t, s);
        lds_barrier();
        gate_math(0, t);
        store_h(0, t);
        issue_gather(0, t);
      } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          partials(i, t, s);
          lds_barrier();
          gate_math(i, t);
          // The other tile's gather: tile 1's of step t-1 (for tile 0), tile 0's of step t (for tile 1).
          const int to = i == 0 ? t - 1 : t;
          if (to >= 0 && !complete_gather(1 - i, to, -1)) {
            ok = false;
            break;
          }
          store_h(i, t);
          issue_gather(i, t);
        }
        if (!ok) break;
      }
      if (t + 1 == probe_next) {
        write_probe(probe_i);
        ++probe_i;
        probe_next = probe_i < a.n_probe ? a.probe_steps[probe_i] : -1;
      }
      ++unpublished;
    }
  }
  // Final publication, and the final h of the tile whose last gather is still open (the other
  // tile's completed during that tile's last step) for the head.
  if (ok && Tt > 0) {
    if (has_down) publish(unpublished);
    if (!complete_gather(NTI - 1, Tt - 1, -1)) ok = false;
  }

  if (!ok) {
    if (!has_down && slice == 0 && a.out) {
      for (int idx = threadIdx.x; idx < NTI * 16 * a.O; idx += NT) {
        const int gr = a.row0 + tile0 * 16 + idx / a.O;
        if (gr < a.row_end) a.out[(size_t)gr * a.O + idx % a.O] = (_Float16)__builtin_nanf("");
      }
    }
    return;
  }

  if (!has_down && a.out_seq && active) {
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      if (!row_ok[i]) continue;
      for (int t = Tt; t < a.T; ++t) {
        _Float16* dst = a.out_seq + ((size_t)grow[i] * a.T + t) * a.H + eu;
#pragma unroll
        for (int j = 0; j < 2; ++j)
          if (eu + j < a.H) dst[j] = (_Float16)0.0f;
      }
    }
  }
  while (probe_i < a.n_probe) {
    write_probe(probe_i);
    ++probe_i;
  }
  if (active) {
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      if (!row_ok[i]) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int u = eu + j;
        if (u < a.H) {
          const size_t si = ((size_t)layer * a.B + grow[i]) * a.H + u;
          if (a.h_n) a.h_n[si] = hcur[i][j];
          if (a.c_n) a.c_n[si] = (_Float16)c[i][j];
        }
      }
    }
  }
  // Linear head (last layer, first slice) on the full final h held in hbuf.
  if (!has_down && slice == 0 && a.out) {
    for (int idx = threadIdx.x; idx < NTI * 16 * a.O; idx += NT) {
      const int rt = idx / a.O, o = idx % a.O;
      const int i = rt / 16, rr = rt % 16;
      const int gr = a.row0 + (tile0 + i) * 16 + rr;
      if (gr >= a.row_end) continue;
      const _Float16* hf = reinterpret_cast<const _Float16*>(hbuf[i]);
      const float* wr = a.wlin + (size_t)o * HP;
      float s0 = 0.f, s1 = 0.f;
      for (int k8 = 0; k8 < HP; k8 += 8) {
        const f16x8 hv = *reinterpret_cast<const f16x8*>(hf + frag_index<16>(rr, k8));
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          s0 = fmaf((float)hv[j], wr[k8 + j], s0);
          s1 = fmaf((float)hv[j + 1], wr[k8 + j + 1], s1);
        }
      }
      a.out[(size_t)gr * a.O + o] = (_Float16)(a.blin[o] + (s0 + s1));
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
  using C = Tile<HP, 16, 1>;
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

// Sliced weights: [L][S][8 waves][8 chunks][4 gates][64 lanes][8].  Wave w of slice s holds unit
// group Sliced::group_of(w); member e = Sliced::member_of(w) selects the part e / KSP (0: W_ih,
// 1: W_hh) and the quarter e % KSP of that part's columns.
template <int HP>
__global__ void pack_sliced_kernel(const _Float16* __restrict__ w_ih, const _Float16* __restrict__ w_hh, int K,
                                   int H, _Float16* __restrict__ dst) {
  using C = Sliced<HP>;
  const size_t total = (size_t)C::kS * 8 * 8 * 4 * 64 * 8;
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int j = e & 7;
  const int lane = (e >> 3) & 63;
  const int q = (e >> 9) & 3;
  const int kc = (int)((e >> 11) & 7);
  const int wv = (int)((e >> 14) & 7);
  const int sl = (int)(e >> 17);
  const int g = C::group_of(wv), ew = C::member_of(wv);
  const bool rec = ew >= C::kKsp;
  const int kq = ew % C::kKsp;
  const int u = sl * C::kHs + g * 16 + (lane & 15);
  const size_t col = (size_t)q * H + u;
  const int k = (kq * 8 + kc) * 32 + (lane >> 4) * 8 + j;
  _Float16 v = (_Float16)0.0f;
  if (u < H) {
    if (!rec) {
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

// x [B, T, I] -> xp [ntile][T][kci0][4][rows] f16x8: B-fragment order for tiles of `rows` rows,
// zero padded.
__global__ void pack_x_kernel(const _Float16* __restrict__ x, int T, int I, int row0, int row_end, int ntile,
                              int rows, int kci0, f16x8* __restrict__ xp) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int fv = 4 * rows;
  const size_t total = (size_t)ntile * T * kci0 * fv;
  if (e >= total) return;
  const int f = (int)(e % fv);
  const int kc = (int)((e / fv) % kci0);
  const size_t tt = e / ((size_t)fv * kci0);
  const int t = (int)(tt % T);
  const int tile = (int)(tt / T);
  const int b = row0 + tile * rows + f % rows;
  const int k0 = kc * 32 + (f / rows) * 8;
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
  else if (H <= 256) HP = 256;
  else if (H <= 512) HP = 512;
  if (HP == 0) {
    *why = "hidden_size > 512 is not implemented by the persistent kernels";
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
  g->slices = HP == 256 ? Sliced<256>::kS : HP == 512 ? Sliced<512>::kS : 1;
  g->max_wg_tiles = HP == 256 ? 2 : 1;
  g->waves = g->slices > 1 ? 8 : HP / 16;
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
  // HP / 16 gate-row groups x kc chunks of 64 lanes x 8 halfs per gate: the same size whether one
  // workgroup or `slices` workgroups hold a layer.
  off = align256(off + (size_t)g.L * (g.HP / 16) * g.kc * 4 * 64 * 8 * sizeof(_Float16));
  p.bias = off;
  off = align256(off + (size_t)g.L * 4 * g.HP * sizeof(float));
  p.wlin = off;
  off = align256(off + (size_t)g.O * g.HP * sizeof(float));
  p.blin = off;
  off = align256(off + (size_t)g.O * sizeof(float));
  p.total = off;
  return p;
}

WorkspaceLayout workspace_layout(const Geometry& g, int seq_len, int chunk_rows, int tile_rows) {
  WorkspaceLayout w;
  const size_t ntile = (size_t)chunk_rows / tile_rows;
  const size_t frag_bytes = (size_t)4 * tile_rows * 16;  // one [tile_rows x 32] fp16 fragment block
  w.chunk_rows = chunk_rows;
  w.tile_rows = tile_rows;
  w.status = 0;
  w.counters = 256;
  w.xp = align256(w.counters + sizeof(uint32_t) * (size_t)g.L * ntile);
  w.hseq = align256(w.xp + ntile * seq_len * g.kc_in0 * frag_bytes);
  w.xring = align256(w.hseq + (size_t)(g.L - 1) * ntile * seq_len * g.kci * frag_bytes);
  w.xring_words = g.slices > 1 ? (size_t)g.L * ntile * 2 * g.HP * 8 : 0;
  w.total = align256(w.xring + w.xring_words * sizeof(uint64_t));
  return w;
}

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

hipError_t launch_pack_x(const Geometry& g, const ForwardArgs& a, hipStream_t s) {
  const size_t n = (size_t)a.ntile * a.T * g.kc_in0 * 4 * a.tile_rows;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_x_kernel, blocks_for(n, 256), 256, 0, s, a.x, a.T, a.I, a.row0, a.row_end, a.ntile,
                     a.tile_rows, g.kc_in0, a.xp);
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

template <int ROWS, bool RAGGED>
static const void* recurrent_kernel_rows(int HP) {
  switch (HP) {
    case 32: return reinterpret_cast<const void*>(&lstm_wavefront_kernel<32, ROWS, kChunk, RAGGED>);
    case 64: return reinterpret_cast<const void*>(&lstm_wavefront_kernel<64, ROWS, kChunk, RAGGED>);
    case 128: return reinterpret_cast<const void*>(&lstm_wavefront_kernel<128, ROWS, kChunk, RAGGED>);
    default: return nullptr;
  }
}

// Steps per chunk of the sliced kernels: the input ring holds wg_tiles * CH * HP / 32 fragment
// blocks and each thread stages its share of one chunk in VGPRs.
constexpr int kChunk256 = 4;
constexpr int kChunk256x2 = 2;
constexpr int kChunk512 = 2;

static const void* recurrent_kernel(const Geometry& g, int tile_rows, bool ragged, int wg_tiles = 1) {
  if (g.slices > 1) {
    if (tile_rows != 16) return nullptr;
    switch (g.HP) {
      case 256:
        return wg_tiles == 2 ? reinterpret_cast<const void*>(&lstm_sliced_kernel<256, kChunk256x2, 2>)
                             : reinterpret_cast<const void*>(&lstm_sliced_kernel<256, kChunk256, 1>);
      case 512: return wg_tiles == 1 ? reinterpret_cast<const void*>(&lstm_sliced_kernel<512, kChunk512, 1>) : nullptr;
      default: return nullptr;
    }
  }
  if (tile_rows == 8) return ragged ? recurrent_kernel_rows<8, true>(g.HP) : recurrent_kernel_rows<8, false>(g.HP);
  if (tile_rows == 16) return ragged ? recurrent_kernel_rows<16, true>(g.HP) : recurrent_kernel_rows<16, false>(g.HP);
  return nullptr;
}

int recurrent_capacity(const Geometry& g, int tile_rows, hipError_t* err) {
  // The smallest occupancy of the variants (with and without lengths, every tile count), so any fits.
  int cap = 0;
  for (int v = 0; v < 2 * g.max_wg_tiles; ++v) {
    const bool ragged = v & 1;
    const void* fn = recurrent_kernel(g, tile_rows, ragged, 1 + v / 2);
    if (!fn) {
      *err = hipErrorInvalidValue;
      return 0;
    }
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, g.waves * 64, 0);
    *err = e;
    if (e != hipSuccess) return 0;
    cap = (cap == 0 || per_cu * cus < cap) ? per_cu * cus : cap;
  }
  return cap;
}

hipError_t launch_recurrent(const Geometry& g, const ForwardArgs& a, hipStream_t s) {
  const void* fn = recurrent_kernel(g, a.tile_rows, a.lengths != nullptr, a.wg_tiles);
  if (!fn || a.wg_tiles < 1 || a.ntile % a.wg_tiles) return hipErrorInvalidValue;
  ForwardArgs args = a;
  void* params[] = {&args};
  return hipLaunchCooperativeKernel(fn, dim3(a.L * a.ntile / a.wg_tiles * g.slices), dim3(g.waves * 64), params, 0,
                                    s);
}

}  // namespace plh
