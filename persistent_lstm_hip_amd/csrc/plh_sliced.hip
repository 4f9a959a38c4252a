// plh_sliced.hip -- the persistent sliced kernel (H 129..512) of the stacked LSTM + Linear
// inference forward on CDNA4 (gfx950).
//
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
// coherent across the XCDs' L2 caches without cache maintenance; when all slices of a group run on
// one XCD (checked at entry) the words are stored without sc1 and stay in its L2 (same_xcd_group).  Two ring slots suffice: a slice
// can overwrite slot t % 2 with h_{t+2} only after it has read h_{t+1} of every sibling, and a
// sibling writes h_{t+1} only after it has read h_t from every slice.  The ring is zeroed before
// each launch (tags start at 1).
//
// Hand-off to the next layer: h is also stored to the hand-off buffer with agent-scope relaxed
// stores; at the end of each chunk every thread waits for its stores to complete (s_waitcnt)
// before the barrier that precedes a relaxed counter increment.  The next layer reads the buffer
// with ordinary loads after an agent-scope acquire, which invalidates any stale copy in its L2.
#include "plh_device.h"

namespace plh {
namespace {

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
  __shared__ int s_l2;

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
  // Wait for the resident weights here: otherwise the compiler keeps them "possibly outstanding"
  // into the step loop and puts vmcnt waits before the input waves' MFMAs, which (one in-order
  // counter on gfx950) then wait for the gather loads those MFMAs are meant to overlap.
  __builtin_amdgcn_s_waitcnt(0);
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
  const int per = has_up ? KCH * FV : a.g_in0 * 16;  // input f16x8 per step in the source
  const size_t hstep = (size_t)KCH * FV;
  const int tile0 = tgrp * NTI;  // first 16-row tile of this workgroup
  auto in_seq = [&](int i) -> const f16x8* {
    return has_up ? a.hseq + ((size_t)(layer - 1) * a.ntile + tile0 + i) * a.T * hstep
                  : a.xp + (size_t)(tile0 + i) * a.T * per;
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
  // A step's source holds the first `per` of its KCH * FV ring entries (layer 0: the g_in0 8-wide K
  // groups of x; the rest of the ring stays zero from the initialisation).
  auto load_chunk = [&](int k) {
    const int s0 = k * CH;
    const int nel = min(CH, Tt - s0) * per;
#pragma unroll
    for (int i = 0; i < NTI; ++i) {
      const f16x8* src = in_seq(i) + (size_t)s0 * per;
#pragma unroll
      for (int r = 0; r < RN; ++r) {
        const int idx = threadIdx.x + r * NT;
        if (idx < nel) R[i][r] = src[idx];
      }
    }
  };
  auto store_chunk = [&](int k) {
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

  // Ring accesses.  Two-tile workgroups run out of VGPRs with global atomics, which hold a 64-bit
  // VGPR address per word; they use buffer loads and stores instead: a descriptor of one ring slot
  // (uniform, in SGPRs), the thread's byte offset in a VGPR and the word's block offset as the
  // scalar offset, with cache policy sc1 (agent-scope coherent, as agent-scope relaxed atomics).
  // Every offset stays inside the slot.  One-tile workgroups keep the global atomics: the extra
  // SGPR pressure of the descriptors costs them more than the VGPRs save.  Descriptor word 3 is
  // 0x00020000: DATA_FORMAT = 32 bit, which untyped buffer accesses need to be non-zero on CDNA.
  auto ring_rs = [&](int i, int t) {
    return __builtin_amdgcn_make_buffer_rsrc(xr(i) + (size_t)(t & 1) * C::kWords, 0, C::kWords * 8, 0x00020000);
  };
  auto gload = [&](int i, int t, int r) -> uint64_t {
    if constexpr (NTI == 2) {
      return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(ring_rs(i, t), threadIdx.x * 8u, r * NT * 8, 16));
    } else {
      return load_agent_u64(xr(i) + (size_t)(t & 1) * C::kWords + threadIdx.x + r * NT);
    }
  };
  // Gather words of tile i, step t: issued right after the tile's own words are stored.
  uint64_t wv[NTI][NW];
  auto issue_gather = [&](int i, int t) {
#pragma unroll
    for (int r = 0; r < NW; ++r) wv[i][r] = gload(i, t, r);
  };
  // Complete the gather of tile i, step t, into hbuf[i]: re-poll the words whose tag is not t + 1
  // yet.  Before spinning, the input waves compute tile i's partials for step t + 1 (ring slot
  // s_next; -1: none).  False (uniformly) if any wait of the workgroup failed.
  auto complete_gather = [&](int i, int t, int s_next) -> bool {
    if (!recurrent && s_next >= 0) partials(i, t + 1, s_next);
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
      if constexpr (NTI == 2) asm volatile("" ::: "memory");  // the buffer loads re-read the ring every spin
#pragma unroll
      for (int r = 0; r < NW; ++r)
        if (word_tag(wv[i][r]) != want) wv[i][r] = gload(i, t, r);
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
    const uint64_t word = tag_word(hcur[i][0], hcur[i][1], (uint32_t)t + 1u);
    // XCD-local groups store the word without sc1 (it stays in their L2), others with it.
    if constexpr (NTI == 2) {
      const auto wd = __builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned int, word);
      if (l2)
        __builtin_amdgcn_raw_buffer_store_b64(wd, ring_rs(i, t), (uint32_t)woff * 8u, 0, 1);
      else
        __builtin_amdgcn_raw_buffer_store_b64(wd, ring_rs(i, t), (uint32_t)woff * 8u, 0, 16);
    } else {
      if (l2)
        __hip_atomic_store(xr(i) + (size_t)(t & 1) * C::kWords + woff, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      else
        __hip_atomic_store(xr(i) + (size_t)(t & 1) * C::kWords + woff, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (has_down) {
      union { _Float16 h[2]; uint32_t u; } v;
      v.h[0] = hcur[i][0];
      v.h[1] = hcur[i][1];
      if constexpr (NTI == 2) {
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(my_seq(i) + (size_t)t * hstep, 0, (int)(hstep * 16), 0x00020000);
        __builtin_amdgcn_raw_buffer_store_b32(v.u, rs, (uint32_t)hoff * 2u, 0, 16);
      } else {
        __hip_atomic_store(reinterpret_cast<uint32_t*>(reinterpret_cast<_Float16*>(my_seq(i) + (size_t)t * hstep) + hoff),
                           v.u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (!has_down && a.out_seq && row_ok[i]) {
      _Float16* dst = a.out_seq + ((size_t)grow[i] * a.T + t) * a.H + eu;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (eu + j < a.H) dst[j] = live ? hcur[i][j] : (_Float16)0.0f;
    }
  };

  int probe_i = 0;
  // Probe steps live in SGPRs (see the wavefront kernel): a VGPR loaded in the loop would put a
  // vmcnt(0) on every step.
  int probe_next = a.n_probe > 0 ? __builtin_amdgcn_readfirstlane(a.probe_steps[0]) : -1;
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

  bool ok = __builtin_amdgcn_readfirstlane(s_fail) == 0;
  if (ok && Tt > 0) {
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
  // Two-tile workgroups: the upstream polls before the loop load into VGPRs that the compiler
  // otherwise treats as possibly outstanding at the loop head, which put a vmcnt(0) (waiting for
  // the other tile's gather) in front of every tile-step's MFMAs.  One wait here costs the first
  // chunk's prefetch once (measured: C3 6.2 -> 5.7 ms; with one tile it is 2% slower, so only
  // two-tile workgroups take it).
  if constexpr (NTI == 2) __builtin_amdgcn_s_waitcnt(0);
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
        probe_next = probe_i < a.n_probe ? __builtin_amdgcn_readfirstlane(a.probe_steps[probe_i]) : -1;
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
    // A wait failed: poison every output of this workgroup (states, probes, output sequence, head).
    if (active) {
#pragma unroll
      for (int i = 0; i < NTI; ++i)
        if (row_ok[i]) poison_lane_outputs(a, layer, grow[i], eu, 2, !has_down);
    }
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

}  // namespace

// Steps per chunk of the sliced kernels: the input ring holds wg_tiles * CH * HP / 32 fragment
// blocks and each thread stages its share of one chunk in VGPRs.
constexpr int kChunk256 = 4;
constexpr int kChunk256x2 = 2;
constexpr int kChunk512 = 2;

const void* sliced_kernel(int HP, int wg_tiles) {
  switch (HP) {
    case 256:
      return wg_tiles == 2 ? reinterpret_cast<const void*>(&lstm_sliced_kernel<256, kChunk256x2, 2>)
                           : reinterpret_cast<const void*>(&lstm_sliced_kernel<256, kChunk256, 1>);
    case 512: return wg_tiles == 1 ? reinterpret_cast<const void*>(&lstm_sliced_kernel<512, kChunk512, 1>) : nullptr;
    default: return nullptr;
  }
}

}  // namespace plh
