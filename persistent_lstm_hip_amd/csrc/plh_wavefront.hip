// plh_wavefront.hip -- the persistent layer-wavefront kernel (H <= 128) of the stacked LSTM +
// Linear inference forward on CDNA4 (gfx950).  Every workgroup of a launch is co-resident (the host
// sizes the grid to the device's occupancy) and loops over the time steps itself.
//
// One workgroup per (layer, batch tile of 8 or 16 rows):
//   * each wave owns 16 hidden units and keeps the i, f, g, o rows of [W_ih | W_hh] for them in
//     VGPRs for the whole sequence as fp16 MFMA A fragments (256 KB per layer at H = 128);
//   * per step a wave computes gates^T[64 gate cols, 16 cols] = W[64, K] * [in_t | h_{t-1}]^T with
//     v_mfma_f32_16x16x32_f16 (fp32 accumulate, bias as the initial accumulator); with 8-row tiles
//     the B columns 8..15 repeat rows 0..7 and each lane evaluates two of its four (unit, row)
//     pairs; the next step's input part is issued between this step's gate computations;
//   * the gate nonlinearities and the c/h update run on the accumulator registers; c never leaves
//     VGPRs; h goes to an LDS history (double-buffered by chunk) that also feeds the next step's
//     recurrent MFMAs and the hand-off copy;
//   * activations live in "fragment order": a [R rows x 32 k] block is stored as [k/8][row][8],
//     i.e. exactly the B operand of one MFMA (lane l reads 16 B at l * 16), in LDS and in the
//     global hand-off buffer, so LDS traffic is conflict-free and global traffic contiguous;
//   * the step input (x for layer 0, h of layer l-1 otherwise) reaches LDS one chunk of CH steps at
//     a time into a double-buffered ring, loaded four steps before it is needed, so no step waits
//     on global memory;
//   * the hand-off between layers is a per-(layer, tile) step counter: the h of each chunk goes to
//     the hand-off buffer with agent-scope (sc1) stores, and once every wave's stores completed the
//     counter is advanced with a relaxed store (no L2 write-back); the next layer polls it and reads
//     the chunk after an agent-scope acquire.  All per-chunk work sits on fixed steps of the chunk
//     (the step body is inlined per step), so there is no chunk-boundary barrier and layer l+1 runs
//     about two chunks behind layer l;
//   * the Linear head runs in the last layer's epilogue on the final h held in LDS;
//   * every wait between workgroups is bounded in wall-clock time; a failed wait sets a status bit,
//     fails every other wait and poisons the outputs, so the grid always drains.
//
// Reference behaviour restated (mantuoluozk/persistent_lstm_hip): gate order i, f, g, o and the
// c/h recurrence of persistent_lstm_reference.cpp:21-35; fp16 h storage per step and fp32 c of
// persistent_lstm_hip.cu:520-525; the fp32-accumulated head of persistent_lstm_hip.cu:1662-1682.
#include "plh_device.h"

namespace plh {
namespace {

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

// LDS of one workgroup.  Ring and history are double-buffered by chunk parity, so chunk k+1's
// inputs can be written and chunk k-1's h copied out while chunk k runs.
template <int HP, int ROWS, int CH>
struct WavefrontLds {
  using C = Tile<HP, ROWS, CH>;
  f16x8 ring[2 * CH * C::kKci * C::kFragVec];  // step inputs: chunk k in buffer k & 1
  f16x8 hist[2 * CH * C::kKcr * C::kFragVec];  // h of every step: step (k, s) in buffer k & 1, slot s
  int ok;
  int tlen;
};

// The persistent layer-wavefront recurrence of one (layer, tile).  Template: padded hidden size HP,
// batch rows per workgroup ROWS (16, or 8 with the MFMA's B columns 8..15 duplicating rows 0..7 so
// each lane evaluates two (unit, row) pairs instead of four), steps per hand-off chunk CH, RAGGED:
// rows may end before the tile's last step (lengths given; without it every row is live at every
// step and the state-freezing selects are compiled out), and IN0: the input part is a single K
// chunk (layer 0 with I <= 32), so the input MFMAs on the other, all-zero chunks are skipped.
template <int HP, int ROWS, int CH, bool RAGGED, bool IN0>
__device__ __forceinline__ void wavefront_body(const ForwardArgs& a, WavefrontLds<HP, ROWS, CH>& lds, int layer,
                                               int tile) {
  using C = Tile<HP, ROWS, CH>;
  constexpr int KCI = C::kKci, KCR = C::kKcr, KC = C::kKc, NT = C::kThreads, FV = C::kFragVec;
  constexpr int KIN = IN0 ? 1 : KCI;  // input-part K chunks with MFMA work
  constexpr int UPL = C::kUpl, RN = C::kRn;
  static_assert(CH >= 4 && (CH & (CH - 1)) == 0, "the hand-off schedule needs a power-of-two chunk of >= 4 steps");
  constexpr int kRingBuf = CH * KCI * FV;  // f16x8 per ring buffer (one chunk of step inputs)
  constexpr int kHistBuf = CH * KCR * FV;  // f16x8 per history buffer (one chunk of h)
  f16x8* const ring = lds.ring;
  f16x8* const hist = lds.hist;
  int& s_ok = lds.ok;
  int& s_tlen = lds.tlen;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;            // B-operand / D column
  const int kg = lane >> 4;           // K group of the A/B fragments, row group of D
  const int r = n & (ROWS - 1);       // batch row in the tile
  const int fl = kg * ROWS + r;       // this lane's B fragment within a block

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
      for (int q = 0; q < 4; ++q) w[kc][q] = (kc < KIN || kc >= KCI) ? wp[(kc * 4 + q) * 64] : f16x8{};
  }
  // D rows of this lane: units u0 .. u0+3 of row n; it evaluates UPL of them, starting at uo.
  const int u0 = wave * 16 + kg * 4;
  const int ibase = (ROWS == 8 && n >= 8) ? 2 : 0;
  const int uo = u0 + ibase;
  f32x4 bias[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) bias[q] = *reinterpret_cast<const f32x4*>(a.bias + ((size_t)layer * 4 + q) * HP + u0);

  // Initial state (nn.LSTM hx) or zeros; h_{-1} is step CH-1 of "chunk -1" (history buffer 1).
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
  auto hist_h = [&](int t) -> _Float16* {
    return reinterpret_cast<_Float16*>(hist + ((t / CH) & 1) * kHistBuf + (t % CH) * (KCR * FV)) + hoff;
  };
  *reinterpret_cast<hvec*>(hist_h(2 * CH - 1)) = hcur;

  const bool has_up = layer > 0;
  const bool has_down = layer < a.L - 1;
  const int per = has_up ? KCI * FV : a.g_in0 * ROWS;  // input f16x8 per step in the source
  const size_t hstep = (size_t)KCR * FV;     // f16x8 per (tile, step) in the hand-off buffer
  const f16x8* in_seq = has_up ? a.hseq + ((size_t)(layer - 1) * a.ntile + tile) * a.T * hstep
                               : a.xp + (size_t)tile * a.T * per;
  f16x8* out_seq_h = has_down ? a.hseq + ((size_t)layer * a.ntile + tile) * a.T * hstep : nullptr;
  const uint32_t* up_ctr = has_up ? a.counters + (layer - 1) * a.ntile + tile : nullptr;
  uint32_t* my_ctr = a.counters + layer * a.ntile + tile;
  const int sync_tid = C::kWaves > 1 ? 64 : 0;  // the lane that polls upstream (wave 1)

  const int nchunk = (Tt + CH - 1) / CH;
  // Chunk k's step inputs: loaded into VGPRs (R) 4 steps before they are needed, written to ring
  // buffer k & 1 at step CH - 2.  Thread positions are ring positions; a step's source holds the
  // first `per` of its KCI * FV ring entries (layer 0: the g_in0 8-wide K groups of x, the rest stay
  // zero from the initialisation).  Every lane loads (indices clamped into the chunk), so the loads
  // write R directly.
  f16x8 R[RN];
  // A full chunk of a full-width source (layers >= 1) needs no clamping or lane conditions (8-row
  // tiles; the 16-row kernel has no VGPRs for a second copy of these paths).
  const bool full_width = ROWS == 8 && per == KCI * FV;
  auto load_chunk = [&](int k) {
    const int ns_k = min(CH, Tt - k * CH);
    const f16x8* src = in_seq + (size_t)k * CH * per;
    if (full_width && ns_k == CH) {
#pragma unroll
      for (int i = 0; i < RN; ++i) R[i] = src[(int)threadIdx.x + i * NT];
      return;
    }
#pragma unroll
    for (int i = 0; i < RN; ++i) {
      const int p = (int)threadIdx.x + i * NT;
      const int st = min(p / (KCI * FV), ns_k - 1), e = min(p % (KCI * FV), per - 1);
      R[i] = src[st * per + e];
    }
  };
  auto store_chunk = [&](int k) {
    const int ns_k = min(CH, Tt - k * CH);
    f16x8* rb = ring + (k & 1) * kRingBuf;
    if (full_width && ns_k == CH) {
#pragma unroll
      for (int i = 0; i < RN; ++i) rb[(int)threadIdx.x + i * NT] = R[i];
      return;
    }
#pragma unroll
    for (int i = 0; i < RN; ++i) {
      const int p = (int)threadIdx.x + i * NT;
      if (p / (KCI * FV) < ns_k && p % (KCI * FV) < per) rb[p] = R[i];
    }
  };
  // Hand-off copy of chunk k's h history (LDS) to the global sequence buffer: one 16-byte sc1 buffer
  // store per thread and element, so a wave's store instruction writes one contiguous 1 KB run (sc1
  // stores are written through; they become visible to other CUs and XCDs once complete, with no L2
  // write-back).  The descriptor's size is the chunk's valid bytes: the stores of a partial chunk's
  // idle lanes fall outside it and are dropped.
  auto copy_out = [&](int k) {
    const int nv = min(CH, Tt - k * CH) * (KCR * FV);  // valid f16x8 of the chunk
    const f16x8* hb = hist + (k & 1) * kHistBuf;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(out_seq_h + (size_t)k * CH * hstep, 0, nv * 16, 0x00020000);
    f16x8 v[RN];
#pragma unroll
    for (int i = 0; i < RN; ++i) v[i] = hb[min((int)threadIdx.x + i * NT, kHistBuf - 1)];
#pragma unroll
    for (int i = 0; i < RN; ++i)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v[i]),
                                             rs, (uint32_t)((int)threadIdx.x + i * NT) * 16u, 0, 16);
  };
  auto need_for = [&](int k) -> uint32_t { return (uint32_t)min((k + 1) * CH, Tt); };  // chunk k published

  int probe_i = 0;
  // Probe steps are wave-uniform and kept in SGPRs (readfirstlane right after the load): a VGPR
  // loaded in the loop would make the compiler wait for every outstanding global access (vmcnt(0),
  // in order on gfx950, so the chunk loads and the hand-off stores included) at each step.
  int probe_next = a.n_probe > 0 ? __builtin_amdgcn_readfirstlane(a.probe_steps[0]) : -1;
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

  for (int i = threadIdx.x; i < 2 * kRingBuf; i += NT) ring[i] = f16x8{};
  __syncthreads();

  bool ok = true;
  if (Tt > 0) {
    if (has_up) {
      if (threadIdx.x == sync_tid) s_ok = wait_counter(up_ctr, need_for(0), a.status, a.wait_ticks);
      __syncthreads();
      ok = s_ok != 0;
    }
    if (ok) {
      load_chunk(0);
      wait_vmem_all();
      store_chunk(0);
    }
  }
  __syncthreads();  // ring buffer 0 and the initial h visible

  // Hand-off schedule, by step s of chunk k (each step ends with the LDS barrier):
  //   s = 0       copy chunk k-1's h (history buffer (k-1) & 1) to the hand-off buffer with sc1
  //               stores; the polling lane reads the upstream counter (for chunk k+1)
  //   s = 1       every wave waits for its hand-off stores; the polling lane checks the counter
  //               (bounded wait if chunk k+1 is not yet published, then an agent-scope acquire)
  //               and shares the verdict through LDS
  //   s = 2       publish chunk k-1 (relaxed counter store: the stores of every wave completed
  //               before the barrier of step 1); load chunk k+1's inputs into VGPRs
  //   s = CH - 2  write them into ring buffer (k+1) & 1, read from step CH - 1 on
  // so layer l+1 runs two chunks and two steps behind layer l and no step waits on global memory.
  const bool hi = ibase != 0;
  uint32_t poll = 0;
  f32x4 acc_next[4];
  if (ok && Tt > 0) {
    const f16x8* xr = ring + fl;
    f16x8 xv[KIN];
#pragma unroll
    for (int kc = 0; kc < KIN; ++kc) xv[kc] = xr[kc * FV];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc_next[q] = bias[q];
#pragma unroll
    for (int kc = 0; kc < KIN; ++kc)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc_next[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][q], xv[kc], acc_next[q], 0, 0, 0);
  }
  // One step (t = k * CH + s).  Inlined with constant s for the steps of full chunks, so the
  // hand-off schedule costs no branches on the other steps; returns false if a wait failed.
  auto step = [&](const int t, const int s, const int k, const bool more) __attribute__((always_inline)) -> bool {
    if (s == 0) {
      if (has_down && k > 0) copy_out(k - 1);
      if (has_up && more && threadIdx.x == sync_tid)
        poll = __hip_atomic_load(up_ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (s == 2) {
      // Nothing the step needs is outstanding here.  Without this explicit wait the compiler
      // keeps the chunk loads "possibly outstanding" (their consumers, the ring writes, are
      // lane-conditional) and waits for every access in flight -- the counter store below
      // included -- before the recurrent LDS reads that reuse those registers.
      wait_vmem_all();
      if (has_down && k > 0 && threadIdx.x == 0)
        __hip_atomic_store(my_ctr, (uint32_t)(k * CH), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (more && has_up && s_ok == 0) return false;
      load_chunk(more ? k + 1 : k);
    }

    f32x4 acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = acc_next[q];
    // Recurrent part: h_{t-1} from the history slot of the previous step.
    const f16x8* hr = hist + (((t + 2 * CH - 1) / CH) & 1) * kHistBuf + ((t + CH - 1) % CH) * (KCR * FV) + fl;
    f16x8 hv[KCR];
#pragma unroll
    for (int kr = 0; kr < KCR; ++kr) hv[kr] = hr[kr * FV];
#pragma unroll
    for (int kr = 0; kr < KCR; ++kr)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[KCI + kr][q], hv[kr], acc[q], 0, 0, 0);

    // Next step's input part (the last step recomputes a discarded in-range step), interleaved
    // with this step's gate math so the matrix core runs while the VALU evaluates the gates
    // (in-order issue would otherwise queue all VALU work behind a burst of MFMAs).
    const int tn = min(t + 1, Tt - 1);
    const f16x8* xr = ring + ((tn / CH) & 1) * kRingBuf + (tn % CH) * (KCI * FV) + fl;
    f16x8 xv[KIN];
#pragma unroll
    for (int kc = 0; kc < KIN; ++kc) xv[kc] = xr[kc * FV];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc_next[q] = bias[q];
    const bool live = t < len;
    auto input_mfma = [&](int m) __attribute__((always_inline)) {
      const int kc = m / 4, q = m % 4;
      acc_next[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][q], xv[kc], acc_next[q], 0, 0, 0);
    };
    // this lane's pair j: D element ibase + j of every gate tile (one v_cndmask each)
    auto cell_pair = [&](int j) __attribute__((always_inline)) {
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
    };
    if constexpr (ROWS == 8 && RAGGED) {
      // With ragged rows (the selects on `live` add VALU work) the gate math goes first and the
      // next step's input MFMAs follow it: 1.7-2.3% faster than the interleave below, which is
      // the faster one without them.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < UPL; ++j) cell_pair(j);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < KIN * 4; ++m) input_mfma(m);
      __builtin_amdgcn_sched_barrier(0);
    } else if constexpr (ROWS == 8) {
      // Two pairs per lane (~80 VALU instructions per wave): one MFMA, then three VALU
      // instructions, and so on, so both waves of a SIMD keep the matrix core fed and neither
      // queues its gate math behind a burst of MFMAs.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < KIN * 4; ++m) input_mfma(m);
#pragma unroll
      for (int j = 0; j < UPL; ++j) cell_pair(j);
#pragma unroll
      for (int m = 0; m < KIN * 4; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
      }
      __builtin_amdgcn_sched_barrier(0);
    } else {
      // Four pairs per lane: each pair is preceded by its share of the MFMAs and fenced.
      constexpr int kMfmaPerPiece = (KIN * 4 + UPL - 1) / UPL;
#pragma unroll
      for (int j = 0; j < UPL; ++j) {
#pragma unroll
        for (int m = j * kMfmaPerPiece; m < (j + 1) * kMfmaPerPiece && m < KIN * 4; ++m) input_mfma(m);
        cell_pair(j);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    *reinterpret_cast<hvec*>(hist_h(t)) = hcur;
    if (!has_down && a.out_seq && row_ok) {
      _Float16* dst = a.out_seq + ((size_t)grow * a.T + t) * a.H + uo;
#pragma unroll
      for (int j = 0; j < UPL; ++j)
        if (uo + j < a.H) dst[j] = live ? hcur[j] : (_Float16)0.0f;
    }
    if (t + 1 == probe_next) {
      write_probe(probe_i);
      ++probe_i;
      probe_next = probe_i < a.n_probe ? __builtin_amdgcn_readfirstlane(a.probe_steps[probe_i]) : -1;
    }
    if (s == 1) {
      // Hand-off stores of step 0 complete before the barrier, so the counter published at step 2
      // covers every wave's stores.
      if (has_down && k > 0) __builtin_amdgcn_s_waitcnt(0);
      if (has_up && more && threadIdx.x == sync_tid) {
        const uint32_t need = need_for(k + 1);
        int okv;
        if (poll >= need) {
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
          okv = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u ? 1 : 0;
        } else {
          okv = wait_counter(up_ctr, need, a.status, a.wait_ticks);
        }
        s_ok = okv;
      }
    } else if (s == CH - 2) {
      wait_vmem_all();  // chunk k+1's inputs, on every path (the ring writes are lane-conditional)
      if (more) store_chunk(k + 1);
    }
    lds_barrier();
    return true;
  };
  const int nfull = Tt / CH;
  for (int k = 0; ok && k < nfull; ++k) {
    const bool more = k + 1 < nchunk;
#pragma unroll
    for (int s = 0; s < CH; ++s)
      if (!step(k * CH + s, s, k, more)) {
        ok = false;
        break;
      }
  }
  for (int t = nfull * CH; ok && t < Tt; ++t)
    if (!step(t, t - nfull * CH, nfull, false)) ok = false;

  if (!ok) {
    // A hand-off wait failed (the status word records it and fails every other wait): poison every
    // output of this workgroup (states, probes, output sequence, head) and leave.
    if (row_ok) poison_lane_outputs(a, layer, grow, uo, UPL, !has_down);
    if (!has_down && a.out) {
      for (int idx = threadIdx.x; idx < ROWS * a.O; idx += NT) {
        const int g = a.row0 + tile * ROWS + idx / a.O;
        if (g < a.row_end) a.out[(size_t)g * a.O + idx % a.O] = (_Float16)__builtin_nanf("");
      }
    }
    return;
  }
  if (has_down && Tt > 0) {
    copy_out(nchunk - 1);
    __builtin_amdgcn_s_waitcnt(0);  // every wave's hand-off stores complete before the counter moves
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(my_ctr, (uint32_t)Tt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    const _Float16* hf = reinterpret_cast<const _Float16*>(hist + (((Tt - 1 + 2 * CH) / CH) & 1) * kHistBuf +
                                                           ((Tt - 1 + 2 * CH) % CH) * (KCR * FV));
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


// One workgroup per (layer, tile).  Layer 0 with x inside one 32-wide K chunk (I <= 32: at most 4
// 8-wide K groups) takes the IN0 body, chosen once here, so no step of either body branches on it.
template <int HP, int ROWS, int CH, bool RAGGED>
__global__ void __launch_bounds__(HP / 16 * 64)
lstm_wavefront_kernel(ForwardArgs a) {
  __shared__ WavefrontLds<HP, ROWS, CH> lds;
  int layer, tile;
  block_coords(blockIdx.x, a.ntile, a.xcd_map, layer, tile);
  if (layer == 0 && a.g_in0 <= 4)
    wavefront_body<HP, ROWS, CH, RAGGED, true>(a, lds, layer, tile);
  else
    wavefront_body<HP, ROWS, CH, RAGGED, false>(a, lds, layer, tile);
}

}  // namespace

// Steps per hand-off chunk: 16 with 8-row tiles at padded H <= 64, where a step is short and the
// per-chunk work weighs more than the longer lag between layers (H64 L2 B512 -5.4%, H32 L8 -3.9%;
// at H 128 it was slower, C2 +0.9%, C5 +1.3%, and with 16-row tiles it does not fit the LDS);
// 8 otherwise.
template <int HP, int ROWS>
constexpr int chunk_steps() { return ROWS == 8 && HP <= 64 ? 16 : 8; }

template <int ROWS, bool RAGGED>
static const void* wavefront_kernel_rows(int HP) {
  switch (HP) {
    case 32: return reinterpret_cast<const void*>(&lstm_wavefront_kernel<32, ROWS, chunk_steps<32, ROWS>(), RAGGED>);
    case 64: return reinterpret_cast<const void*>(&lstm_wavefront_kernel<64, ROWS, chunk_steps<64, ROWS>(), RAGGED>);
    case 128: return reinterpret_cast<const void*>(&lstm_wavefront_kernel<128, ROWS, chunk_steps<128, ROWS>(), RAGGED>);
    default: return nullptr;
  }
}

const void* wavefront_kernel(int HP, int tile_rows, bool ragged) {
  if (tile_rows == 8) return ragged ? wavefront_kernel_rows<8, true>(HP) : wavefront_kernel_rows<8, false>(HP);
  if (tile_rows == 16) return ragged ? wavefront_kernel_rows<16, true>(HP) : wavefront_kernel_rows<16, false>(HP);
  return nullptr;
}

}  // namespace plh
