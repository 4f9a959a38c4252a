// plh_device.h -- device-side building blocks shared by the gfx950 kernels: vector types, the LSTM
// cell update, LDS and inter-workgroup synchronisation, the MFMA fragment order, and the work
// split of the sliced kernels (which their weight packer must reproduce).
#pragma once

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
// The minimum is IEEE 754-2019 `minimum` (v_minimum3_f32), which returns NaN for a NaN argument, so a
// NaN pre-activation gives a NaN gate as torch does (fminf would return the cap).
constexpr float kExpCap = 40.0f;
__device__ __forceinline__ float exp_neg(float z, float k) {
  return __builtin_amdgcn_exp2f(__builtin_elementwise_minimum(z * (-k * kLog2e), kExpCap));
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

// s_waitcnt on the vector-memory counter alone (vmcnt = 0; expcnt and lgkmcnt at their no-wait
// maxima in the gfx9 encoding).  gfx950 retires loads and stores on this counter in issue order.
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Barrier that orders LDS traffic only: global stores stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Spin (one lane) until *ctr >= need, bounded by `limit` ticks of s_memrealtime (100 MHz), then
// acquire at agent scope.  Returns 0 if the wait timed out or any workgroup of the grid has failed.
__device__ __attribute__((unused)) int wait_counter(const uint32_t* ctr, uint32_t need, uint32_t* status, uint64_t limit) {
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

// After a failed wait: NaN into every output element a lane owns, units u0 + stride * j (j < n) of
// batch row `grow` in `layer`: h_n, c_n, every probe and, for the last layer, every step of out_seq.
// With the head poisoned as well, each output element of a forward is then either its correct value
// or NaN.
__device__ __attribute__((unused)) void poison_lane_outputs(const ForwardArgs& a, int layer, int grow, int u0, int n,
                                                            bool last, int stride = 1) {
  const float qnan = __builtin_nanf("");
  const _Float16 hnan = (_Float16)qnan;
  for (int j = 0; j < n; ++j) {
    const int u = u0 + stride * j;
    if (u >= a.H) continue;
    const size_t si = ((size_t)layer * a.B + grow) * a.H + u;
    if (a.h_n) a.h_n[si] = hnan;
    if (a.c_n) a.c_n[si] = hnan;
    for (int p = 0; p < a.n_probe; ++p) {
      const size_t o = (((size_t)p * a.L + layer) * a.B + grow) * a.H + u;
      a.probe_h[o] = qnan;
      a.probe_c[o] = qnan;
    }
    if (last && a.out_seq)
      for (int t = 0; t < a.T; ++t) a.out_seq[((size_t)grow * a.T + t) * a.H + u] = hnan;
  }
}

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

// Work split of the sliced kernels (H 129..512): S workgroups ("slices") per (layer, 16-row tile),
// each holding the gate rows of HS hidden units for both the layer input and h.  Wave w of a slice
// owns 4 NJ units (HS = 32 NJ) over all of K: NJ MFMA A tiles of 16 gate rows each (row r of tile j
// is gate r % 4 of unit 4 NJ w + 4 j + r / 4) for 2 KCH K-chunks, KCH of W_ih then KCH of W_hh,
// i.e. 2 KCH NJ = 32 fragments (128 VGPRs) at both padded sizes.
template <int HP>
struct Sliced {
  static constexpr int kS = HP == 256 ? 4 : 16;  // workgroups per (layer, tile)
  static constexpr int kHs = HP / kS;            // hidden units per workgroup: 64 or 32
  static constexpr int kNj = kHs / 32;           // A tiles per wave: 2 or 1
  static constexpr int kKch = HP / 32;           // K chunks of the layer input and of h
  static constexpr int kWords = HP * 8;          // ring words reserved per step slot of a tile (the
                                                 // packed words of one step take half)
  static_assert(HP == 256 || HP == 512, "padded H 256 or 512");
};

// Work split of the layer-sequential recurrent kernel (plh_rec.hip): the input projection comes
// precomputed, so a workgroup holds only W_hh rows, for HS hidden units, and S workgroups
// ("slices") serve a 16-row tile.  Wave w serves the 4 NJ units 4 NJ w .. + 4 NJ - 1 of its slice
// over all of K as NJ MFMA A tiles of 16 gate rows (row r of tile j: gate r % 4 of unit
// 4 NJ w + 4 j + r / 4), KCH K-chunks of 32 each, i.e. KCH NJ fragments (4 VGPRs each):
//   HP     NJ  HS  S   fragments per wave
//   128    2   64  2   8
//   256    2   64  4   16
//   512    2   64  8   32  (128 VGPRs)
//   1024   1   32  32  32  (128 VGPRs; 32 slices = the 32 CUs of one XCD per tile)
template <int HP>
struct Rec {
  static constexpr int kNj = HP == 1024 ? 1 : 2;  // A tiles (4-unit groups) per wave
  static constexpr int kUpw = 4 * kNj;    // hidden units per wave
  static constexpr int kHs = 8 * kUpw;    // hidden units per workgroup
  static constexpr int kS = HP / kHs;     // workgroups per 16-row tile
  static constexpr int kKch = HP / 32;    // K chunks of h
  static constexpr int kWords = HP * 8;   // ring words reserved per step slot of a tile (the packed
                                          // words of one step take half)
  static_assert(HP == 128 || HP == 256 || HP == 512 || HP == 1024, "padded H of the layer-sequential path");
  static_assert(kS * kHs == HP && kS >= 2 && kS <= 32, "slices");
};
// Rec<HP>::kS for a runtime padded H (host side).
inline int rec_slices(int HP) { return HP == 1024 ? 32 : HP / 64; }

// ---- tagged exchange of h among the workgroups of a tile (plh_sliced.hip; plh_rec.hip shares
// sliced_coords and packs its words itself) ----

// Packed exchange words.  A 64-bit word carries 4 fp16 h of one batch row and a 4-bit step tag, one
// tag bit in bit 14 (the exponent's top bit) of each fp16.  That bit is clear in every h a step
// computes (|h| <= 1 < 2); NaN and infinity, the only other values with it set, travel as +-1.5
// (never an h) and come back as NaN.  The bit is cleared in every value sent, so the tag is always
// intact.  Rows of length 0 keep their h0, which may use the bit: their exchanged values only feed
// their own frozen rows, and the kernels restore h0 before it is read as a result.
// The xw_* helpers are also host functions, so that a host program can check them exhaustively.
typedef unsigned short xw_u16x2 __attribute__((ext_vector_type(2)));
typedef short xw_s16x2 __attribute__((ext_vector_type(2)));
// Two fp16 (bit patterns, low and high half) made exchange-safe: a half with an all-ones exponent
// (NaN, infinity) becomes sign | 0x3E00 (+-1.5), every other half loses bit 14.  Per half, the
// exponent bits plus 0x0400 carry into bit 15 exactly when they are all ones; an arithmetic shift
// makes that a mask of the half, and one bit-field insert picks marker or value.  Packed 16-bit
// operations for both halves (v_pk_add_u16, v_pk_ashrrev_i16, v_bfi_b32) instead of a compare and
// select each.
__host__ __device__ __forceinline__ uint32_t xw_enc_pair(uint32_t p) {
  const xw_u16x2 f = __builtin_bit_cast(xw_u16x2, p & 0x7C007C00u) + xw_u16x2{0x0400, 0x0400};
  uint32_t special = __builtin_bit_cast(uint32_t, __builtin_bit_cast(xw_s16x2, f) >> (short)15);
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("" : "+v"(special));  // keeps the mask a mask (else it is rebuilt as per-half compares and selects)
#endif
  return (special & ((p & 0x80008000u) | 0x3E003E00u)) | (~special & p & 0xBFFFBFFFu);
}
// Two fp16 of a word back, the tag bits cleared and +-1.5 restored as NaN.  Per 16-bit half, m (the
// value without sign and tag bit) is <= 0x3C00 for every h (|h| <= 1) and 0x3E00 for the marker;
// adding 0x4300 sets bit 15 exactly when m >= 0x3D00 (1.25), and that bit, moved to bit 14, turns
// the marker into NaN (0x7E00) where the tag bit was.  One packed 16-bit add for both halves instead
// of a compare and select each.  (Values 1.25 <= |x| < 2 other than the marker, which only the
// frozen rows of length 0 can carry, also come back as NaN; those rows' h is restored from h0.)
__host__ __device__ __forceinline__ uint32_t xw_dec_pair(uint32_t v) {
  const xw_u16x2 z = __builtin_bit_cast(xw_u16x2, v & 0x3FFF3FFFu) + xw_u16x2{0x4300, 0x4300};
  return (v & 0xBFFFBFFFu) | ((__builtin_bit_cast(uint32_t, z) >> 1) & 0x40004000u);
}
__host__ __device__ __forceinline__ uint32_t xw_tag(uint64_t w) {
  return (uint32_t)(((w >> 14) & 1u) | ((w >> 29) & 2u) | ((w >> 44) & 4u) | ((w >> 59) & 8u));
}
// True if the tag bits of word w are want_bits (= xw_tag_bits of the wanted tag): one masked compare
// of the 64-bit word instead of gathering its four tag bits.
__host__ __device__ __forceinline__ bool xw_tag_is(uint64_t w, uint64_t want_bits) {
  return ((w ^ want_bits) & 0x4000400040004000ull) == 0u;
}
__host__ __device__ __forceinline__ uint64_t xw_tag_bits(uint32_t tag) {
  return ((uint64_t)(tag & 1u) << 14) | ((uint64_t)((tag >> 1) & 1u) << 30) | ((uint64_t)((tag >> 2) & 1u) << 46) |
         ((uint64_t)((tag >> 3) & 1u) << 62);
}
// Tag of step t's words in a two-slot ring (slot t & 1): successive writes to a slot (steps t - 2
// and t) differ, and none is 0 (the cleared ring).
__host__ __device__ __forceinline__ uint32_t xw_step_tag(int t) { return (uint32_t)((t >> 1) % 15) + 1u; }

__device__ __forceinline__ uint64_t load_agent_u64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// XCD-local exchange.  A store without the sc1 bit (a workgroup-scope relaxed atomic store) writes
// through the CU's L1 into its XCD's L2 and stays there; the exchange's polls (sc1 buffer loads)
// bypass the reader's L1 and read that L2.  Between CUs of one XCD this hand-off is visible and a
// round trip costs ~1070 cycles instead of ~1360 for agent-scope stores, which write through to
// memory (MI355X, one wave per CU); across XCDs such a store is never seen, so it may only be used
// when every workgroup of the exchange runs on the same XCD.  Tags guard correctness either way: a
// reader only takes a word whose tag is the current step's.
__device__ __forceinline__ uint32_t xcc_id() {
  return __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u;  // HW_REG_XCC_ID, bits 3:0
}

// Thread 0 of each of the n workgroups of an exchange group: publish this XCD's id in table[self]
// (agent scope; the table is zeroed before the launch) and wait, bounded by wait_ticks, for the
// other entries.  Returns 1 if all n run on this XCD, 0 if not, -1 if the wait timed out (status
// set).  Every member sees the same n entries, so all take the same decision.
__device__ __forceinline__ int same_xcd_group(uint32_t* table, int self, int n, uint32_t* status,
                                              uint64_t wait_ticks) {
  const uint32_t mine = xcc_id() + 1u;
  __hip_atomic_store(table + self, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  int same = 1;
  for (int s = 0; s < n; ++s) {
    uint32_t v;
    while ((v = __hip_atomic_load(table + s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0u) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > wait_ticks) {
        __hip_atomic_fetch_or(status, PLH_STATUS_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return -1;
      }
    }
    same &= v == mine;
  }
  return same;
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

}  // namespace
}  // namespace plh
