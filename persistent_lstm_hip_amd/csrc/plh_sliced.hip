// plh_sliced.hip -- the persistent sliced kernel (H 129..512) of the stacked LSTM + Linear
// inference forward on CDNA4 (gfx950).
//
// Hidden sizes above 128.  A layer's [W_ih | W_hh] (1 MB at H = 256, 4 MB at H = 512) no longer fits
// one CU's register file, so each (layer, 16-row tile) is served by S workgroups ("slices"), each
// keeping the gate rows of HS = HP / S hidden units resident in VGPRs (Sliced<HP>):
//   * wave w of a slice owns 4 NJ units over all of K (the layer input and h): its A tiles
//     interleave the gates (row r: gate r % 4 of unit 4 j + r / 4), so the D fragments give each
//     lane all four gates of its units eu + 4 j for one row, and the cell update needs no other
//     wave: no partial sums cross waves;
//   * a step's gate sums are one MFMA chain per tile that starts from the bias: the input part
//     x_t W_ih^T is computed a step ahead (off the critical path, from the layer input staged in
//     LDS), and only h_{t-1} W_hh^T (KCH NJ MFMAs per wave) sits between a step's exchange and its
//     cell update;
//   * the slices exchange h_t every step through a two-slot ring of tagged 64-bit words (the xw_*
//     words of plh_device.h: 4 fp16 and a 4-bit step tag each); a reader polls every slice's
//     words (its own included) until their tags are the step's, with no counter or barrier between
//     a slice's cell update and its siblings' next step.  When the S slices of a group run on one
//     XCD (checked at entry) the words are stored without sc1 and stay in its L2 (same_xcd_group);
//   * with two tiles per workgroup (NTI = 2) a step computes both tiles, so its fixed costs (the
//     exchange's round trip, the memory issue of eight waves, one workgroup barrier) are paid once
//     per two tiles;
//   * layers run as a wavefront.  h_t also goes to the hand-off buffer (hseq, fragment order, sc1
//     stores); each wave publishes its stores per group of G steps with one atomic add to the
//     (layer, tile) counter, and the next layer's waves check that counter (prefetched a step
//     ahead) before they load an input step, D steps before it is used, in 1 KB pieces staged
//     through registers into a two-slot LDS ring.
//
// Memory ordering rests on gfx950 retiring loads and stores on one counter in issue order: a wave
// that has waited for its latest ring poll has also completed everything it issued before that
// poll (its earlier hand-off stores, the input piece and the counter value it prefetched), so no
// extra wait sits on the step.
//
// Reference behaviour restated (mantuoluozk/persistent_lstm_hip): the generic path's recurrence
// (persistent_lstm_hip.cu:2923-3181) with the input projection kept in fp32, gate order i, f, g, o
// and the c/h recurrence of persistent_lstm_reference.cpp:21-35.
#include "plh_device.h"

namespace plh {
namespace {

template <int HP, int NTI>
__global__ void __launch_bounds__(512) lstm_sliced_kernel(ForwardArgs a) {
  using C = Sliced<HP>;
  constexpr int S = C::kS, HS = C::kHs, KCH = C::kKch, NJ = C::kNj;
  constexpr int NT = 512, FV = 64;        // 16-row fragment blocks: 64 lanes x 16 bytes
  constexpr int UPW = 4 * NJ;             // hidden units per wave
  constexpr int KW = 4 / NJ;              // lanes with kgx % KW == 0 send a word
  constexpr int SB = 4 * HS;              // packed words of one slice per step
  constexpr int PW = S * SB;              // packed words of one step of a tile (4 HP)
  constexpr int NLD = PW / 2 / NT;        // 16-byte poll loads per thread and step
  constexpr int D2 = NJ == 2 ? 2 : 1;     // u32 distance in hbuf between a word's two pairs
  constexpr int SW = HP == 256 ? 4 : 8;   // waves that stage the input pieces
  constexpr int BPW = KCH / SW;           // 1 KB input blocks each of them stages per step
  constexpr int G = 2;                    // steps per publication of the hand-off
  constexpr int D = 3;                    // steps between an input's load and its use
  constexpr uint32_t kOutOfRange = 0x80000000u;  // buffer offset past every range: stores dropped
  static_assert(NTI == 1 || NTI == 2, "one or two tiles per workgroup");
  static_assert(PW % (2 * NT) == 0 && KCH % 8 == 0, "whole loads per thread");

  // h of tile i in fragment order, double-buffered by step: step t reads h_{t-1} from hbuf[i][t & 1]
  // and gathers h_t into hbuf[i][(t + 1) & 1].
  __shared__ f16x8 hbuf[NTI][2][KCH * FV];
  __shared__ f16x8 ring[NTI][2][KCH * FV];  // layer input x_t of tile i in slot t & 1
  __shared__ float s_bias[4][HS];
  __shared__ int s_fail;
  __shared__ int s_tlen;
  __shared__ int s_l2;
  __shared__ uint32_t s_up[NTI];  // upstream counter of tile i as last read by wave 0

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int layer, tgrp, slice;
  sliced_coords(blockIdx.x, a.ntile / NTI, S, a.xcd_map, layer, tgrp, slice);
  // Workgroups of the groups that only round the grid up to a multiple of 8 (whole groups per XCD).
  if (layer >= a.L) return;
  const int en = lane & 15, kgx = lane >> 4;
  // This lane's units eu + 4 j (j < NJ) of row en: all four gates of each are in its D fragments.
  const int eu = slice * HS + wave * UPW + kgx;
  const bool writer = kgx % KW == 0;
  const int tile0 = tgrp * NTI;  // first 16-row tile of this workgroup
  const bool has_up = layer > 0;
  const bool has_down = layer + 1 < a.L;

  int grow[NTI], len[NTI];
  bool row_ok[NTI];
  if (threadIdx.x == 0) {
    s_tlen = 0;
    s_fail = 0;
    // Zeroed before the first barrier: every staging wave reads it in the prologue, and LDS keeps
    // what an earlier workgroup left there (a stale upstream count would let a wave load hand-off
    // steps that are not yet published).
    for (int i = 0; i < NTI; ++i) s_up[i] = 0;
    // With xcd_map the S slices of a (layer, tile group) are dispatched to one XCD; checked here,
    // and only then do they exchange h through that XCD's L2 (same_xcd_group; the table of the
    // groups' XCD ids follows the rings).
    s_l2 = 0;
    if (a.xcd_map) {
      uint32_t* table = reinterpret_cast<uint32_t*>(a.xring + (size_t)a.L * a.ntile * 2 * C::kWords) +
                        ((size_t)layer * (a.ntile / NTI) + tgrp) * S;
      const int r = same_xcd_group(table, slice, S, a.status, a.wait_ticks);
      if (r < 0) s_fail = 1;
      s_l2 = r > 0;
    }
  }
  __syncthreads();
  const bool l2 = __builtin_amdgcn_readfirstlane(s_l2) != 0;
#pragma unroll
  for (int i = 0; i < NTI; ++i) {
    grow[i] = a.row0 + (tile0 + i) * 16 + en;
    row_ok[i] = grow[i] < a.row_end;
    len[i] = 0;
    if (row_ok[i]) {
      len[i] = a.lengths ? a.lengths[grow[i]] : a.T;
      len[i] = len[i] < 0 ? 0 : (len[i] > a.T ? a.T : len[i]);
    }
    if (wave == 0 && lane < 16) atomicMax(&s_tlen, len[i]);
  }
  __syncthreads();
  // Steps of this workgroup: the longest row of its tiles (the same in every layer).
  const int Tt = __builtin_amdgcn_readfirstlane(s_tlen);

  // Resident weights: chunks 0 .. KCH - 1 of W_ih, then KCH of W_hh, NJ tiles each.
  f16x8 w[2 * KCH][NJ];
  {
    const f16x8* wp = reinterpret_cast<const f16x8*>(a.wpack) +
                      (size_t)((layer * S + slice) * 8 + wave) * 2 * KCH * NJ * 64 + lane;
#pragma unroll
    for (int kc = 0; kc < 2 * KCH; ++kc)
#pragma unroll
      for (int j = 0; j < NJ; ++j) w[kc][j] = wp[(kc * NJ + j) * 64];
  }
  // The resident weights complete here (otherwise the compiler keeps them "possibly outstanding"
  // and waits for every global access in flight before the step loop's MFMAs).
  __builtin_amdgcn_s_waitcnt(0);
  for (int idx = threadIdx.x; idx < 4 * HS; idx += NT) {
    const int q = idx / HS, u = idx % HS;
    s_bias[q][u] = a.bias[((size_t)layer * 4 + q) * HP + slice * HS + u];
  }

  float c[NTI][NJ];
  _Float16 hcur[NTI][NJ];
#pragma unroll
  for (int i = 0; i < NTI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int u = eu + 4 * j;
      const bool v = row_ok[i] && u < a.H;
      const size_t si = ((size_t)layer * a.B + grow[i]) * a.H + u;
      c[i][j] = (v && a.c0) ? (float)a.c0[si] : 0.0f;
      hcur[i][j] = (v && a.h0) ? a.h0[si] : (_Float16)0.0f;
    }
  // h_{-1} of all units into hbuf (fragment order), and a zero input ring.
  auto fill_h0 = [&](int i, f16x8* dst) {
    for (int idx = threadIdx.x; idx < KCH * FV; idx += NT) {
      const int kc = idx / FV, l = idx % FV;
      const int gr = a.row0 + (tile0 + i) * 16 + (l & 15);
      const int k0 = kc * 32 + (l >> 4) * 8;
      f16x8 v = {};
      if (a.h0 && gr < a.row_end) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (k0 + j < a.H) v[j] = a.h0[((size_t)layer * a.B + gr) * a.H + k0 + j];
      }
      dst[idx] = v;
    }
  };
#pragma unroll
  for (int i = 0; i < NTI; ++i) fill_h0(i, hbuf[i][0]);
  for (int idx = threadIdx.x; idx < NTI * 2 * KCH * FV; idx += NT)
    ring[idx / (2 * KCH * FV)][(idx / (KCH * FV)) & 1][idx % (KCH * FV)] = f16x8{};
  __syncthreads();  // s_bias, hbuf and the ring complete

  // b_ih + b_hh of this lane's units by gate, in registers for the whole sequence.
  float bias[4][NJ];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int j = 0; j < NJ; ++j) bias[q][j] = s_bias[q][wave * UPW + kgx + 4 * j];

  // ---- layer input: staged into the LDS ring in 1 KB pieces, D steps ahead ----
  // The pieces are loaded unconditionally (lanes past the input address it out of range), so that
  // every path of a step issues the same loads.
  const int per = has_up ? KCH * FV : a.g_in0 * 16;  // f16x8 per step in the source
  const size_t hstep = (size_t)KCH * FV;
  // Descriptor of tile i's input of step s (word 3 0x00020000: DATA_FORMAT = 32 bit, which untyped
  // buffer accesses need on CDNA).
  // Step-0 addresses of each tile's input and hand-off sequences (a step is `per`, resp. hstep,
  // f16x8 further), computed once.
  const f16x8* in_base[NTI];
  f16x8* out_base[NTI];
#pragma unroll
  for (int i = 0; i < NTI; ++i) {
    in_base[i] = has_up ? a.hseq + ((size_t)(layer - 1) * a.ntile + tile0 + i) * a.T * hstep
                        : a.xp + (size_t)(tile0 + i) * a.T * per;
    out_base[i] = a.hseq + ((size_t)layer * a.ntile + tile0 + i) * a.T * hstep;
  }
  auto in_rs = [&](int i, int s) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<f16x8*>(in_base[i] + s * per), 0, per * 16, 0x00020000);
  };
  // Waves 0 .. SW - 1 stage the input.  At padded H 256 these are the first waves of the SIMDs,
  // which finish a step's work earlier (the matrix core serves them first) and would otherwise wait
  // at the step's barrier, while the second waves' part of the step is its critical path (C3 -1.1%,
  // B = 64 -6.7%); at H 512 a step's input is twice as large and all waves stage it (with four, B = 64
  // was 3.2% slower).
  const bool stager = SW == 8 || __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < SW;
  // Input piece of tile i, step s: block wave * BPW + b of the step, one f16x8 per lane.  Entries
  // past `per` (layer 0: x's K groups) read out of the descriptor's range, which returns zero.  The
  // previous layer's h is read with sc1: it was written with sc1 by other CUs, and its counter was
  // seen before the load is issued.
  f16x8 pc[NTI][BPW];
  auto load_piece = [&](int i, int s) {
    if (!stager) return;
    const __amdgpu_buffer_rsrc_t rs = in_rs(i, s);
#pragma unroll
    for (int b = 0; b < BPW; ++b) {
      const uint32_t off = (uint32_t)((wave * BPW + b) * FV + lane) * 16u;
      if (has_up)
        pc[i][b] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 16));
      else
        pc[i][b] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
  };
  auto store_piece = [&](int i, int s) {
    if (!stager) return;
#pragma unroll
    for (int b = 0; b < BPW; ++b) ring[i][s & 1][(wave * BPW + b) * FV + lane] = pc[i][b];
  };

  // ---- hand-off publication and its check by the next layer ----
  // A (layer, tile) counter counts groups of G steps times the S slices: thread 0 of each slice
  // adds a group once its workgroup's hand-off stores of that group are complete.  Wave 0 reads the
  // upstream counter every step (used a step later) and shares it in LDS.
  constexpr int CS = kSlicedCounterStride;
  auto up_ctr = [&](int i) -> uint32_t* { return a.counters + ((size_t)(layer - 1) * a.ntile + tile0 + i) * CS; };
  auto my_ctr = [&](int i) -> uint32_t* { return a.counters + ((size_t)layer * a.ntile + tile0 + i) * CS; };
  int pub[NTI];                   // groups of tile i published (thread 0)
  int avail[NTI];                 // groups of tile i known published upstream (this wave)
  uint32_t cup[NTI];              // wave 0: upstream counter of tile i, loaded a step earlier
#pragma unroll
  for (int i = 0; i < NTI; ++i) {
    pub[i] = 0;
    avail[i] = 0;
    cup[i] = 0;
  }
  auto load_counter = [&](int i) {
    if (has_up && wave == 0) cup[i] = __hip_atomic_load(up_ctr(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  // Thread 0, after a step's barrier: the hand-off stores of tile i's steps < n are complete (each
  // was issued before a poll its wave has waited for).
  auto publish = [&](int i, int n) {
    const int groups = n >= Tt ? (Tt + G - 1) / G : n / G;
    if (groups > pub[i]) {
      if (threadIdx.x == 0)
        __hip_atomic_fetch_add(my_ctr(i), (uint32_t)(groups - pub[i]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pub[i] = groups;
    }
  };
  // Make step s of tile i's input available: its group published upstream.  The shared counter
  // usually shows it; otherwise spin (bounded).  False if the wait failed.
  auto need_input = [&](int i, int s) -> bool {
    const int g = s / G;
    if (g < avail[i]) return true;
    const uint32_t need = (uint32_t)S * (uint32_t)(g + 1);
    // An LDS read (each step's barrier orders it after wave 0's write); through a generic pointer it
    // would be a flat load, whose wait covers every global access in flight.
    uint32_t v = __builtin_amdgcn_readfirstlane(s_up[i]);
    if (v < need) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      for (;;) {
        v = __builtin_amdgcn_readfirstlane(__hip_atomic_load(up_ctr(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (v >= need) break;
        if (__hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return false;
        if (__builtin_amdgcn_s_memrealtime() - t0 > a.wait_ticks) {
          __hip_atomic_fetch_or(a.status, PLH_STATUS_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          return false;
        }
        __builtin_amdgcn_s_sleep(8);
      }
    }
    avail[i] = (int)(v / (uint32_t)S);
    return true;
  };
  auto clamp_step = [&](int s) { return s < Tt ? s : Tt - 1; };

  // ---- MFMA parts of a step ----
  f32x4 acc[NTI][NJ];
  // acc[i] = bias + x_s W_ih^T of tile i (x_s in ring slot s & 1).
  auto input_mfma = [&](int i, int s) {
    const f16x8* src = ring[i][s & 1] + lane;
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{bias[0][j], bias[1][j], bias[2][j], bias[3][j]};
#pragma unroll
    for (int kc = 0; kc < KCH; ++kc) {
      const f16x8 bv = src[kc * FV];
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][j], bv, acc[i][j], 0, 0, 0);
    }
  };
  // acc[i] += h_{t-1} W_hh^T, the h fragments read from LDS four K-chunks ahead of their MFMAs.
  auto rec_mfma = [&](int i, const f16x8* hprev) {
    constexpr int kAhead = 4;
    f16x8 bq[kAhead];
#pragma unroll
    for (int k = 0; k < kAhead; ++k) bq[k] = hprev[k * FV + lane];
#pragma unroll
    for (int kc = 0; kc < KCH; ++kc) {
      const f16x8 bv = bq[kc % kAhead];
      if (kc + kAhead < KCH) bq[kc % kAhead] = hprev[(kc + kAhead) * FV + lane];
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[KCH + kc][j], bv, acc[i][j], 0, 0, 0);
    }
  };
  // Cell update of tile i, step t: element q of acc[i][j] is gate q of unit eu + 4 j.  Both units'
  // updates are computed on every lane and then selected (under a branch on `live` the compiler
  // would serialise the units' dependency chains).
  auto cell = [&](int i, int t) {
    const bool live = t < len[i];
    float cn[NJ], hn[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      cn[j] = c[i][j];
      lstm_cell(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3], cn[j], hn[j]);
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) asm volatile("" : "+v"(cn[j]), "+v"(hn[j]));
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      c[i][j] = live ? cn[j] : c[i][j];
      hcur[i][j] = live ? (_Float16)hn[j] : hcur[i][j];
    }
  };

  // ---- exchange ----
  // Ring of tile i: two slots of C::kWords words (PW used), slot t & 1 for step t; words in writer
  // order [slice][wave][16 NJ]: lane (kgx, en) with kgx % KW == 0 writes word
  // wave * 16 NJ + (kgx / KW) * 16 + en of its slice's block, carrying units (eu, eu + 1) and
  // (eu + 4, eu + 5) (NJ = 2, from itself and lane + 16) or eu .. eu + 3 (NJ = 1, from lanes + 16,
  // + 32, + 48) of row en.
  uint64_t* xr_base[NTI];
#pragma unroll
  for (int i = 0; i < NTI; ++i) xr_base[i] = a.xring + ((size_t)layer * a.ntile + tile0 + i) * 2 * C::kWords;
  auto xr = [&](int i) -> uint64_t* { return xr_base[i]; };
  const int pwoff = slice * SB + wave * 16 * NJ + (kgx / KW) * 16 + en;
  auto slot_rs = [&](int i, int t) {
    return __builtin_amdgcn_make_buffer_rsrc(xr(i) + (size_t)__builtin_amdgcn_readfirstlane(t & 1) * C::kWords, 0,
                                             PW * 8, 0x00020000);
  };
  // LDS destination (u32 index into a fragment-ordered h block) of the first pair of word m of a
  // step; the second pair is D2 further.
  auto word_dst = [](int m) -> int {
    const int sl = m / SB, wq = m % SB;
    const int wv_ = wq / (16 * NJ), rem = wq % (16 * NJ);
    const int u0 = sl * HS + wv_ * UPW + (rem / 16) * KW;
    return ((u0 >> 3) * 16 + (rem & 15)) * 4 + ((u0 & 7) >> 1);
  };
  // Poll p of a thread reads words m and m + 1 of every slice's block: waves 0-3 the words that the
  // slices' waves 0-3 write (the first half of a block), waves 4-7 the other half.  The second wave
  // of each SIMD finishes its MFMAs later (the matrix core serves the older wave first), and so do
  // its words; polled by the waves that are late themselves, they are usually written when polled.
  auto poll_word = [](int tid, int p) -> int {
    const int half = tid / (NT / 2), j = tid % (NT / 2) + p * (NT / 2);
    return (j / (SB / 4)) * SB + half * (SB / 2) + 2 * (j % (SB / 4));
  };
  int gdst[2 * NLD];
#pragma unroll
  for (int r = 0; r < 2 * NLD; ++r) gdst[r] = word_dst(poll_word((int)threadIdx.x, r >> 1) + (r & 1));
  uint64_t wv[NTI][2 * NLD];  // poll results of each tile
  // Poll p of tile i, step t: words poll_word(tid, p) and + 1 of the slot, one 16-byte load with sc1
  // (each word is written by one aligned 8-byte store and lies inside the load, so it is read whole;
  // its own tag validates it).  The offset is a per-wave part (slice and half) plus 16 bytes per lane.
  const uint32_t poll_off = (uint32_t)poll_word((int)threadIdx.x, 0) * 8u;
  auto poll = [&](int i, int t, int p) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(slot_rs(i, t), poll_off, p * (NT / 2) / (SB / 4) * SB * 8, 16);
    wv[i][2 * p] = (uint64_t)v[0] | ((uint64_t)v[1] << 32);
    wv[i][2 * p + 1] = (uint64_t)v[2] | ((uint64_t)v[3] << 32);
  };
  // Tile i's h_t to the siblings: one word from each writer lane (the others address no word).
  auto send = [&](int i, int t) {
    uint32_t lo, hi;
    if constexpr (NJ == 2) {
      const uint32_t mine = (uint32_t)__builtin_bit_cast(uint16_t, hcur[i][0]) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, hcur[i][1]) << 16);
      const uint32_t other = (uint32_t)__builtin_amdgcn_ds_swizzle((int)mine, 0x401F);  // lane ^ 16
      lo = __builtin_amdgcn_perm(other, mine, 0x05040100u);
      hi = __builtin_amdgcn_perm(other, mine, 0x07060302u);
    } else {
      const uint32_t mine = (uint32_t)__builtin_bit_cast(uint16_t, hcur[i][0]);
      const uint32_t other = (uint32_t)__builtin_amdgcn_ds_swizzle((int)mine, 0x401F);  // lane ^ 16
      lo = __builtin_amdgcn_perm(other, mine, 0x05040100u);
      hi = (uint32_t)__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, (int)lo);             // lane + 32's pair
    }
    const uint64_t word = (uint64_t)xw_enc_pair(lo) | ((uint64_t)xw_enc_pair(hi) << 32) | xw_tag_bits(xw_step_tag(t));
    const auto wd = __builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned int, word);
    const uint32_t woff = writer ? (uint32_t)pwoff * 8u : kOutOfRange;
    // XCD-local groups store without sc1 (the word stays in their L2), others with it.
    if (l2)
      __builtin_amdgcn_raw_buffer_store_b64(wd, slot_rs(i, t), woff, 0, 1);
    else
      __builtin_amdgcn_raw_buffer_store_b64(wd, slot_rs(i, t), woff, 0, 16);
  };
  // The polls of tile i's step t, issued after the tile's word and (two tiles) the other tile's cell
  // update, when the siblings' words are usually written: a poll that finds a stale word costs a
  // round trip at the gather.  Loads and stores retire in issue order, so the gather's wait covers
  // nothing issued after these loads.
  auto issue_poll = [&](int i, int t) {
#pragma unroll
    for (int p = 0; p < NLD; ++p) poll(i, t, p);
  };
  // Complete the gather of tile i, step t, into dst: re-poll the words whose tag is not step t's
  // yet (bounded wait; a failure sets s_fail), then scatter them into fragment order.
  auto gather = [&](int i, int t, f16x8* dst) {
    const uint64_t want = xw_tag_bits(xw_step_tag(t));
    uint64_t t0 = 0;
    for (int spin = 0;; ++spin) {
      // & rather than &&: every word is tested (no lane-masked branch per word)
      bool ready = true;
#pragma unroll
      for (int r = 0; r < 2 * NLD; ++r) ready = ready & xw_tag_is(wv[i][r], want);
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
      asm volatile("" ::: "memory");  // the re-polls are not loop-invariant loads
#pragma unroll
      for (int p = 0; p < NLD; ++p)
        if (!(xw_tag_is(wv[i][2 * p], want) & xw_tag_is(wv[i][2 * p + 1], want))) poll(i, t, p);
    }
    uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
#pragma unroll
    for (int r = 0; r < 2 * NLD; ++r) {
      d32[gdst[r]] = xw_dec_pair((uint32_t)wv[i][r]);
      d32[gdst[r] + D2] = xw_dec_pair((uint32_t)(wv[i][r] >> 32));
    }
  };
  // The loads of this wave's previous step for tile i (input piece, counter) were issued before
  // the polls it has just waited for, so they are complete: the empty asm tells the compiler, which
  // would otherwise wait for them as loads in flight where they are read.
  auto settle = [&](int i) {
#pragma unroll
    for (int b = 0; b < BPW; ++b) asm volatile("" : "+v"(pc[i][b]));
    asm volatile("" : "+v"(cup[i]));
  };

  // Hand-off to the next layer: h_s of tile i, this slice's HS units, from its fragment-ordered h
  // block to the hand-off buffer (the same order), one 16-byte sc1 store per thread of waves 0 ..
  // HS / 32 - 1, a step after the gather that completed it.
  constexpr int CPY = HS / 32 * FV;  // f16x8 of a slice's units per step
  auto copy_out = [&](int i, int s_, const f16x8* src) {
    if (!has_down || (int)threadIdx.x >= CPY) return;
    const int idx = slice * CPY + (int)threadIdx.x;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(out_base[i] + s_ * (int)hstep, 0, (int)(hstep * 16), 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, src[idx]),
                                           rs, (uint32_t)idx * 16u, 0, 16);
  };
  // The last layer's output sequence (issued before the step's ring poll, as it is optional).
  auto store_out_seq = [&](int i, int t) {
    if (has_down || !a.out_seq || !row_ok[i]) return;
    const bool live = t < len[i];
    _Float16* dst = a.out_seq + ((size_t)grow[i] * a.T + t) * a.H + eu;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (eu + 4 * j < a.H) dst[4 * j] = live ? hcur[i][j] : (_Float16)0.0f;
  };

  int probe_i = 0;
  // Probe steps live in SGPRs (a VGPR loaded in the loop would put a vmcnt(0) on every step).
  int probe_next = a.n_probe > 0 ? __builtin_amdgcn_readfirstlane(a.probe_steps[0]) : -1;
  auto write_probe = [&](int pi) {
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      if (!row_ok[i]) continue;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int u = eu + 4 * j;
        if (u < a.H) {
          const size_t o = (((size_t)pi * a.L + layer) * a.B + grow[i]) * a.H + u;
          a.probe_h[o] = (float)hcur[i][j];
          a.probe_c[o] = c[i][j];
        }
      }
    }
  };

  // ---- prologue: inputs of steps 0 and 1 into the ring, step 2 into the piece registers, the
  // upstream counter, and the first step's input part ----
  bool ok = __builtin_amdgcn_readfirstlane(s_fail) == 0;
  if (ok && Tt > 0) {
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      if (has_up && stager && !need_input(i, clamp_step(D - 1))) ok = false;
      if (!ok) break;
#pragma unroll
      for (int s = 0; s < D - 1; ++s) {
        load_piece(i, clamp_step(s));
        wait_vmem_all();
        store_piece(i, s);
      }
      load_piece(i, clamp_step(D - 1));
      load_counter(i);
    }
    if (!ok) s_fail = 1;
  }
  wait_vmem_all();
  __syncthreads();
  ok = __builtin_amdgcn_readfirstlane(s_fail) == 0;
  if (ok && Tt > 0) {
#pragma unroll
    for (int i = 0; i < NTI; ++i) input_mfma(i, 0);
  }
  lds_barrier();  // step 0 overwrites ring slot 0 (with x_2) once every wave has read x_0

  // ---- steps ----
  // Step t, for both tiles of a two-tile workgroup at once (the exchange's round trip, the memory
  // issue and the barrier are paid once per step, not per tile): h_{t-1} W_hh^T; each tile's cell
  // update, output sequence and word; the polls of step t, each followed by one tile's input part
  // x_{t+1} W_ih^T, which covers the round trip (a poll issued right after the tile's own word would
  // often find the siblings' words not yet written); the gathers into the other h buffer; then,
  // off the step's chain, the input of step t + 2 into the ring, the hand-off copy of h_{t-1}, the
  // input pieces of step t + 3 and the counter (issued after the gathers, so that no wait of this
  // step covers them); one barrier, after which thread 0 publishes.
  for (int t = 0; ok && t < Tt; ++t) {
#pragma unroll
    for (int i = 0; i < NTI; ++i) rec_mfma(i, hbuf[i][t & 1]);
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      cell(i, t);
      store_out_seq(i, t);
      send(i, t);
    }
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      if constexpr (NTI == 2) issue_poll(i, t);
      if (t + 1 < Tt) input_mfma(i, t + 1);
      if constexpr (NTI == 1) issue_poll(i, t);
    }
#pragma unroll
    for (int i = 0; i < NTI; ++i) gather(i, t, hbuf[i][(t + 1) & 1]);
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      settle(i);
      store_piece(i, t + 2);
      if (t > 0) copy_out(i, t - 1, hbuf[i][t & 1]);
      if (threadIdx.x == 0) s_up[i] = cup[i];
      if (has_up && stager && !need_input(i, clamp_step(t + D))) s_fail = 1;
      load_piece(i, clamp_step(t + D));
      load_counter(i);
    }
    lds_barrier();
    if (has_down) {
#pragma unroll
      for (int i = 0; i < NTI; ++i) publish(i, t - 1);
    }
    if (__builtin_amdgcn_readfirstlane(s_fail) != 0) {
      ok = false;
      break;
    }
    if (t + 1 == probe_next) {
      write_probe(probe_i);
      ++probe_i;
      probe_next = probe_i < a.n_probe ? __builtin_amdgcn_readfirstlane(a.probe_steps[probe_i]) : -1;
    }
  }
  // The last step's hand-off copy and the final publication, once every wave's copies are complete.
  if (ok && Tt > 0) {
#pragma unroll
    for (int i = 0; i < NTI; ++i) copy_out(i, Tt - 1, hbuf[i][Tt & 1]);
    wait_vmem_all();
    __syncthreads();
    ok = __builtin_amdgcn_readfirstlane(s_fail) == 0;
    if (ok && has_down) {
#pragma unroll
      for (int i = 0; i < NTI; ++i) publish(i, Tt);
    }
  }
  auto hfinal = [&](int i) -> f16x8* { return hbuf[i][Tt & 1]; };
  // Rows of length 0 keep their h0, which the packed exchange may not carry intact: restore their
  // h in the final buffer before the head reads it.
  if (ok && a.lengths && Tt > 0) {
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      for (int idx = threadIdx.x; idx < KCH * FV; idx += NT) {
        const int kc = idx / FV, l = idx % FV;
        const int gr = a.row0 + (tile0 + i) * 16 + (l & 15);
        if (gr >= a.row_end || a.lengths[gr] > 0) continue;
        const int k0 = kc * 32 + (l >> 4) * 8;
        f16x8 v = {};
        if (a.h0) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (k0 + j < a.H) v[j] = a.h0[((size_t)layer * a.B + gr) * a.H + k0 + j];
        }
        hfinal(i)[idx] = v;
      }
    }
    __syncthreads();
  }

  if (!ok) {
    // A wait failed: poison every output of this workgroup (states, probes, output sequence, head).
#pragma unroll
    for (int i = 0; i < NTI; ++i)
      if (row_ok[i]) poison_lane_outputs(a, layer, grow[i], eu, NJ, !has_down, 4);
    if (!has_down && slice == 0 && a.out) {
      for (int idx = threadIdx.x; idx < NTI * 16 * a.O; idx += NT) {
        const int gr = a.row0 + tile0 * 16 + idx / a.O;
        if (gr < a.row_end) a.out[(size_t)gr * a.O + idx % a.O] = (_Float16)__builtin_nanf("");
      }
    }
    return;
  }

  // Steps past the workgroup's longest row were never visited: their output sequence is zero.
  if (!has_down && a.out_seq) {
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      if (!row_ok[i]) continue;
      for (int t = Tt; t < a.T; ++t) {
        _Float16* dst = a.out_seq + ((size_t)grow[i] * a.T + t) * a.H + eu;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          if (eu + 4 * j < a.H) dst[4 * j] = (_Float16)0.0f;
      }
    }
  }
  while (probe_i < a.n_probe) {
    write_probe(probe_i);
    ++probe_i;
  }
#pragma unroll
  for (int i = 0; i < NTI; ++i) {
    if (!row_ok[i]) continue;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int u = eu + 4 * j;
      if (u < a.H) {
        const size_t si = ((size_t)layer * a.B + grow[i]) * a.H + u;
        if (a.h_n) a.h_n[si] = hcur[i][j];
        if (a.c_n) a.c_n[si] = (_Float16)c[i][j];
      }
    }
  }
  // Linear head (last layer, first slice) on the full final h.
  if (!has_down && slice == 0 && a.out) {
    for (int idx = threadIdx.x; idx < NTI * 16 * a.O; idx += NT) {
      const int rt = idx / a.O, o = idx % a.O;
      const int i = rt / 16, rr = rt % 16;
      const int gr = a.row0 + (tile0 + i) * 16 + rr;
      if (gr >= a.row_end) continue;
      const _Float16* hf = reinterpret_cast<const _Float16*>(hfinal(i));
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

}  // namespace

const void* sliced_kernel(int HP, int wg_tiles) {
  switch (HP) {
    case 256:
      return wg_tiles == 2 ? reinterpret_cast<const void*>(&lstm_sliced_kernel<256, 2>)
                           : reinterpret_cast<const void*>(&lstm_sliced_kernel<256, 1>);
    case 512: return wg_tiles == 1 ? reinterpret_cast<const void*>(&lstm_sliced_kernel<512, 1>) : nullptr;
    default: return nullptr;
  }
}

}  // namespace plh
