// plh_rec.hip -- the layer-sequential path on CDNA4 (gfx950), padded H 128, 256, 512 and 1024.
//
// With [W_ih | W_hh] resident (plh_sliced.hip) a layer of H = 512 needs 16 workgroups per 16-row
// tile, so a 256-CU device covers 64 rows of all layers per launch, and a layer of H = 1024 would not
// fit at all.  Here each layer's input projection for all T steps is one GEMM (x_t W_ih^T, fp16 in
// and out with fp32 accumulation, as the reference's torch::matmul of fp16 tensors; plh_gemm.hip,
// launched by the host) and the persistent kernel below keeps only W_hh resident: S workgroups
// ("slices") per 16-row tile, HS hidden units each (the Rec<HP> table of plh_device.h: 8 slices of
// 64 units at H = 512, 32 slices of 32 units at H = 1024), so one launch covers 512 rows of one
// layer at H = 512 and 128 rows at H = 1024.  The layers run one after another.  This path also
// serves input sizes above the padded hidden size (any H), whose layer-0 input part the all-layers
// kernels cannot hold.  Layer 0 with I <= 32 (H 512, 1024) needs no GEMM: its x_t W_ih^T is one K
// chunk of MFMAs inside the kernel (the X0 variant), from x packed in B-fragment order, so nothing
// of size T x rows x 4H is written.
//   * the GEMM's output columns are in lane order: W_ih's rows are permuted (and padded to 4 HP) at
//     pack time so that the projections one lane needs per step (4 gates x NJ units) are 8 NJ
//     contiguous bytes, one load, issued a step ahead; projections and layer inputs are kept
//     fragment-blocked (1 KB per 16 rows x 32 columns), so a wave's projection load and the
//     GEMM's stores and loads each move contiguous 1 KB blocks;
//   * wave w of a slice holds the i, f, g, o rows of W_hh for its 4 NJ units over all of K, as NJ
//     16-row tiles whose rows interleave the gates (row r: gate r % 4 of unit 4 j + r / 4): KCH
//     K-chunks x NJ tiles of MFMA A fragments (128 VGPRs at H 512 and 1024);
//   * per step each wave computes its gate sums from h_{t-1} in LDS (KCH NJ MFMAs in two independent
//     chains: one per tile, or at NJ = 1 the even and the odd K chunks) and each lane then holds all
//     four gates of its units for one row, so the cell update needs no other wave: no partial sums
//     and no barrier between a wave's MFMAs and its gate math, and one wave of a SIMD updates its
//     cells while the other still runs its MFMAs.  h is double-buffered in LDS by step;
//   * the slices exchange h_t every step through a two-slot ring of tagged 64-bit words, with the
//     protocol of plh_sliced.hip (readers re-poll words until their tags are current) but packed
//     words: 4 fp16 and a 4-bit step tag each, and each workgroup polls only its S - 1 siblings;
//     when the slices of a tile run on one XCD (checked at entry) the words stay in its L2
//     (same_xcd_group: the step's wait for its siblings' words fell from ~2900 to ~1350 cycles at
//     H 512); h_t also goes to the next layer's GEMM input, stored a step later from LDS.
//
// Reference behaviour restated (mantuoluozk/persistent_lstm_hip): the generic path's per-layer
// input projection followed by a persistent recurrence (persistent_lstm_hip.cu:2923-3181, which
// serves 1 <= H <= 1024 and any input size), gate order i, f, g, o and the c/h recurrence of
// persistent_lstm_reference.cpp:21-35.
#include <type_traits>

#include "plh_device.h"

namespace plh {
namespace {

// [L][S][8 waves][KCH chunks][NJ tiles][64 lanes][8]: wave w of slice s holds the W_hh rows of its
// units s HS + UPW w .. + UPW - 1 for all of K; row r of tile j's A fragment is gate r % 4 of unit
// s HS + UPW w + 4 j + r / 4, so the D fragment of tile j gives lane l all four gates of unit
// s HS + UPW w + 4 j + l / 16 for batch row l % 16.
template <int HP>
__global__ void pack_rec_kernel(const _Float16* __restrict__ w_hh, int H, _Float16* __restrict__ dst) {
  using C = Rec<HP>;
  constexpr int NJ = C::kNj, KCH = C::kKch;
  const size_t total = (size_t)C::kS * 8 * KCH * NJ * 64 * 8;
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int jj = e & 7;
  const int lane = (e >> 3) & 63;
  size_t rest = e >> 9;
  const int j = (int)(rest % NJ);
  rest /= NJ;
  const int kc = (int)(rest % KCH);
  rest /= KCH;
  const int wv = (int)(rest & 7);
  const int sl = (int)(rest >> 3);
  const int r = lane & 15;
  const int u = sl * C::kHs + wv * C::kUpw + 4 * j + (r >> 2);
  const int q = r & 3;
  const int k = kc * 32 + (lane >> 4) * 8 + jj;
  dst[e] = (u < H && k < H) ? w_hh[((size_t)q * H + u) * H + k] : (_Float16)0.0f;
}

// Lane order of the projection GEMM's output columns (its W operand's rows): column `col` of a
// [.. x 4 HP] projection holds gate *q of hidden unit *u.
//   NJ = 2: col = ((slice * 8 + wave) * 4 + kgx) * 8 + 2 q + j for unit slice * 64 + 8 wave + kgx + 4 j:
//           lane kgx * 16 + en of that wave reads the 8 halfs of its units (eu, eu + 4) as 16 bytes.
//   NJ = 1: col = ((slice * 4 + wave / 2) * 4 + kgx) * 8 + 4 (wave % 2) + q for unit
//           slice * 32 + 4 wave + kgx: the two waves of a pair share a 32-column block, lane
//           kgx * 16 + en of each reading its 4 halfs (8 bytes) of the lane's 16.
__host__ __device__ inline void rec_lane_column(int col, int HP, int* u, int* q) {
  if (HP == 1024) {
    const int wpar = (col >> 2) & 1, kgx = (col >> 3) & 3, pair = (col >> 5) & 3, slice = col >> 7;
    *q = col & 3;
    *u = slice * 32 + (pair * 2 + wpar) * 4 + kgx;
  } else {
    const int j = col & 1, kgx = (col >> 3) & 3, wave = (col >> 5) & 7, slice = col >> 8;
    *q = (col & 7) >> 1;
    *u = slice * 64 + wave * 8 + kgx + 4 * j;
  }
}

// W_ih ([4H][K], torch layout) as the GEMM's W operand [4 HP][Kp] with rows in lane order
// (rec_lane_column); zero rows for padded units and zero columns K..Kp-1.
__global__ void pack_rec_wih_kernel(const _Float16* __restrict__ w_ih, int H, int HP, int K, int Kp,
                                    _Float16* __restrict__ dst) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (size_t)4 * HP * Kp) return;
  const int col = (int)(e / Kp), k = (int)(e % Kp);
  int u, q;
  rec_lane_column(col, HP, &u, &q);
  dst[e] = (u < H && k < K) ? w_ih[((size_t)q * H + u) * K + k] : (_Float16)0.0f;
}

// W_ih of layer 0 (I <= 32) as MFMA A fragments of the X0 kernel: [S][8 waves][NJ tiles][64 lanes][8],
// tile j's rows as in pack_rec_kernel (gate r % 4 of unit s HS + UPW w + 4 j + r / 4) and
// k = 8 (l / 16) + 0..7.
template <int HP>
__global__ void pack_rec_wx0_kernel(const _Float16* __restrict__ w_ih, int H, int I, _Float16* __restrict__ dst) {
  using C = Rec<HP>;
  constexpr int NJ = C::kNj;
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (size_t)C::kS * 8 * NJ * 64 * 8) return;
  const int jj = e & 7, lane = (e >> 3) & 63;
  size_t rest = e >> 9;
  const int j = (int)(rest % NJ);
  rest /= NJ;
  const int wv = (int)(rest & 7), sl = (int)(rest >> 3);
  const int r = lane & 15;
  const int u = sl * C::kHs + wv * C::kUpw + 4 * j + (r >> 2);
  const int q = r & 3, k = (lane >> 4) * 8 + jj;
  dst[e] = (u < H && k < I) ? w_ih[((size_t)q * H + u) * I + k] : (_Float16)0.0f;
}

// x rows [row0, row_end) into the first GEMM's input, fragment-blocked [T * rows_pad][LD] (row
// t * rows_pad + b): columns 0..KP-1, zero past I and past the launch's rows.
__global__ void rec_input_kernel(const _Float16* __restrict__ x, int T, int I, int row0, int row_end, int rows_pad,
                                 int LD, int KP, _Float16* __restrict__ xs) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (size_t)T * rows_pad * KP) return;
  const int i = (int)(e % KP);
  const size_t tb = e / KP;
  const int b = (int)(tb % rows_pad);
  const int t = (int)(tb / rows_pad);
  const int r = row0 + b;
  xs[blocked_index(tb, i, LD)] = (r < row_end && i < I) ? x[((size_t)r * T + t) * I + i] : (_Float16)0.0f;
}

// X0: layer 0 with I <= 32, its input projection computed here from xp (a.gates unused).
template <int HP, bool X0>
__global__ void __launch_bounds__(512) lstm_rec_kernel(ForwardArgs a) {
  using C = Rec<HP>;
  constexpr int S = C::kS, HS = C::kHs, KCH = C::kKch, NJ = C::kNj, UPW = C::kUpw;
  // K-chunks by which tile 0's MFMA chain leads tile 1's (NJ = 2; see the step), per padded H.
  constexpr int kLead = NJ != 2 ? 0 : HP == 512 ? 8 : HP == 256 ? 4 : 0;
  constexpr int NT = 512, FV = 64;
  constexpr int PW = C::kWords / 2;      // packed words of one step's h of a tile (4 fp16 each)
  constexpr int G = (S - 1) * 2 * HS;    // 16-byte loads of the siblings' words per workgroup and step
  constexpr int NL = (G + NT - 1) / NT;  // loads per thread (at most): 1 at H 128/256, 2 at 512, 4 at 1024
  constexpr int NW = 2 * NL;             // exchange words a thread gathers per step (at most)
  // The step input: a lane's projections (NJ = 2: 8 halfs, NJ = 1: 4 halfs), or under X0 x_t as the
  // lane's MFMA B fragment.
  using GV = std::conditional_t<(X0 || NJ == 2), f16x8, f16x4>;

  // h of all HP units in fragment order, double-buffered by step: step t reads h_{t-1} from buffer
  // t & 1 and writes h_t (its own units and the gathered ones) into the other, so no wave waits for
  // the others between its MFMAs and its gate math.
  __shared__ f16x8 hbuf[2][KCH * FV];
  __shared__ float s_bias[4][HS];
  __shared__ int s_fail;
  __shared__ int s_tlen;
  __shared__ int s_l2;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int grid_layer, tile, slice;
  sliced_coords(blockIdx.x, a.ntile, S, a.xcd_map, grid_layer, tile, slice);
  // Workgroups of the tiles that only round the grid up to a multiple of 8 (whole tiles per XCD).
  if (grid_layer != 0) return;
  const int layer = a.layer;
  const int en = lane & 15, kgx = lane >> 4;
  // This lane's units eu + 4 j (j < NJ) of row en: the D fragments of the wave's tiles (all four
  // gates of unit UPW wave + 4 j + kgx of the slice, row en).
  const int eu = slice * HS + wave * UPW + kgx;
  const int b = tile * 16 + en;  // row within this launch
  const int grow = a.row0 + b;
  const bool row_ok = grow < a.row_end;
  const bool last = a.hout == nullptr;

  if (threadIdx.x == 0) {
    s_tlen = 0;
    // A failed wait of an earlier layer's launch (this forward's status word) fails this one too,
    // so that the head is poisoned whichever layer timed out.
    s_fail = __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
    // With xcd_map the S slices of a tile are dispatched to one XCD (workgroups go round-robin over
    // the XCDs, and theirs are congruent mod 8); checked here, and only then do they exchange h
    // through that XCD's L2 (same_xcd_group; the table follows the ring).
    s_l2 = 0;
    if (a.xcd_map) {
      uint32_t* table = reinterpret_cast<uint32_t*>(a.xring + (size_t)a.ntile * 2 * C::kWords) + tile * S;
      const int r = same_xcd_group(table, slice, S, a.status, a.wait_ticks);
      if (r < 0) s_fail = 1;
      s_l2 = r > 0;
    }
  }
  __syncthreads();
  const bool l2 = __builtin_amdgcn_readfirstlane(s_l2) != 0;
  int len = 0;
  if (row_ok) {
    len = a.lengths ? a.lengths[grow] : a.T;
    len = len < 0 ? 0 : (len > a.T ? a.T : len);
  }
  if (wave == 0 && lane < 16) atomicMax(&s_tlen, len);
  __syncthreads();
  // Steps of this tile: its longest row.  Workgroup-uniform values read from LDS go through
  // readfirstlane, so that the loop's exits are uniform branches the compiler leaves unstructured.
  const int Tt = __builtin_amdgcn_readfirstlane(s_tlen);

  f16x8 w[KCH][NJ];
  {
    const f16x8* wp =
        reinterpret_cast<const f16x8*>(a.wpack) + (size_t)((layer * S + slice) * 8 + wave) * KCH * NJ * 64 + lane;
#pragma unroll
    for (int kc = 0; kc < KCH; ++kc)
#pragma unroll
      for (int j = 0; j < NJ; ++j) w[kc][j] = wp[(kc * NJ + j) * 64];
  }
  // X0: W_ih of layer 0 for the wave's tiles.
  f16x8 wx[NJ] = {};
  if constexpr (X0) {
    const f16x8* p = reinterpret_cast<const f16x8*>(a.wx0) + (size_t)(slice * 8 + wave) * NJ * 64 + lane;
#pragma unroll
    for (int j = 0; j < NJ; ++j) wx[j] = p[j * 64];
  }
  // The resident weights complete here (otherwise the compiler keeps them "possibly outstanding"
  // and waits for every global access in flight before the step loop's MFMAs).
  __builtin_amdgcn_s_waitcnt(0);
  for (int idx = threadIdx.x; idx < 4 * HS; idx += NT) {
    const int q = idx / HS, u = idx % HS;
    s_bias[q][u] = a.bias[((size_t)layer * 4 + q) * HP + slice * HS + u];
  }

  float c[NJ];
  _Float16 hcur[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int u = eu + 4 * j;
    const bool v = row_ok && u < a.H;
    const size_t si = ((size_t)layer * a.B + grow) * a.H + u;
    c[j] = (v && a.c0) ? (float)a.c0[si] : 0.0f;
    hcur[j] = (v && a.h0) ? a.h0[si] : (_Float16)0.0f;
  }
  // h_{-1} of all units of the tile's rows into hbuf (fragment order)
  for (int idx = threadIdx.x; idx < KCH * FV; idx += NT) {
    const int kc = idx / FV, l = idx % FV;
    const int gr = a.row0 + tile * 16 + (l & 15);
    const int k0 = kc * 32 + (l >> 4) * 8;
    f16x8 v = {};
    if (a.h0 && gr < a.row_end) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (k0 + j < a.H) v[j] = a.h0[((size_t)layer * a.B + gr) * a.H + k0 + j];
    }
    hbuf[0][idx] = v;
  }
  __syncthreads();  // hbuf and s_bias complete before the first step (or the head, if no step runs)

  // Input projection of step min(t, Tt - 1) for this lane's row and units, bias excluded: gate q of
  // unit eu + 4 j is element 2 q + j (NJ = 2) or q (NJ = 1).  Padded units read zero columns and
  // padded rows zero inputs.  One unconditional load (a load under an exec branch makes the compiler
  // wait for it together with the ring poll), consumed a step after it is issued.
  // X0: instead, x of step min(t, Tt - 1) as this lane's MFMA B fragment (row en, k 8 kgx .. +7) from
  // xp ([ntile][T][4][16] f16x8).
  // Blocked projections: step t's 16 rows of this tile are block row t * ntile + tile of 4 HP / 32
  // column blocks; this lane's bytes are those of lane kgx * 16 + en of its wave's column block
  // (rec_lane_column).
  constexpr size_t kColBlocks = 4 * HP / 32;
  const f16x8* const xsrc = X0 ? a.xp + (size_t)tile * a.T * 64 + kgx * 16 + en : nullptr;
  const f16x8* const gsrc8 =
      (X0 || NJ != 2) ? nullptr
                      : reinterpret_cast<const f16x8*>(a.gates) + ((size_t)tile * kColBlocks + slice * 8 + wave) * 64 +
                            kgx * 16 + en;
  const f16x4* const gsrc4 =
      (X0 || NJ != 1) ? nullptr
                      : reinterpret_cast<const f16x4*>(a.gates) +
                            (((size_t)tile * kColBlocks + slice * 4 + (wave >> 1)) * 64 + kgx * 16 + en) * 2 + (wave & 1);
  auto gload = [&](int t) -> GV {
    const size_t tc = (size_t)(t < Tt ? t : Tt - 1);
    if constexpr (X0)
      return xsrc[tc * 64];
    else if constexpr (NJ == 2)
      return gsrc8[tc * a.ntile * kColBlocks * 64];
    else
      return gsrc4[tc * a.ntile * kColBlocks * 128];
  };

  // Packed exchange (xw_* words): a word carries 4 units of one row.  NJ = 2: units eu, eu + 1 (low
  // half) and eu + 4, eu + 5 (high half) from a lane with even kgx, which holds eu and eu + 4 and
  // takes eu + 1 and eu + 5 from its partner lane + 16; words in writer order
  // [slice][wave][row en][kgx / 2].  NJ = 1: units 4 w .. 4 w + 3 of the wave from lane kgx = 0,
  // which takes unit +1 from lane + 16 and the pair +2, +3 from lane + 32; words in writer order
  // [slice][wave / 2][row en][wave % 2].  Either way the two words of a 16-byte load are units
  // 8 m .. 8 m + 7 of one row, one f16x8 of h's fragment order.
  uint64_t* ring = a.xring + (size_t)tile * 2 * C::kWords;  // a slot of PW words per step parity
  const int pwoff = NJ == 2 ? (slice * 8 + wave) * 32 + en * 2 + (kgx >> 1)
                            : ((slice * 4 + (wave >> 1)) * 16 + en) * 2 + (wave & 1);  // this lane's word
  const bool writer = NJ == 2 ? (kgx & 1) == 0 : kgx == 0;
  // A workgroup gathers the S - 1 sibling slices' words (its own pairs go to hbuf from registers):
  // load k of thread tid is load index g = 512 k + tid of the step, 2 HS loads per sibling block
  // (the blocks in slice order without this workgroup's own); g < G.  Block and validity are
  // wave-uniform (2 HS and G are multiples of 64).
  // Every thread makes the first G / NT loads; load G / NT exists for the waves below G % NT (a
  // compile-time count and one wave-uniform flag, so the unconditional loads carry no branch).
  constexpr int NLF = G / NT;
  const int wbase = __builtin_amdgcn_readfirstlane((int)threadIdx.x & ~63);
  const bool last_ld = wbase < G - NLF * NT;
  auto has_ld = [&](int k) { return k < NLF || (k == NLF && last_ld); };
  const int q_in = (int)threadIdx.x % (2 * HS);  // load position within a sibling block
  auto sib = [&](int k) {
    const int r = (k * NT + wbase) / (2 * HS);
    return r + (r >= slice ? 1 : 0);
  };
  // hbuf position (f16x8 index) of load k: sibling block sib * 2 HS + q, i.e. units 8 (q / 16) .. + 7
  // of the sibling's block, row q % 16; a wave's loads fill 64 consecutive f16x8 (1 KB), so its one
  // 16-byte LDS store per load is conflict-free.
  auto gdst16 = [&](int k) -> int { return sib(k) * 2 * HS + q_in; };
  // this lane's word's first pair in hbuf (writer lanes): u32 index of units eu, eu + 1
  const int own_dst = ((eu >> 3) * 16 + en) * 4 + ((eu & 7) >> 1);
  // b_ih + b_hh of this lane's units (eu + 4 j) by gate, in registers for the whole sequence.
  float bias[4][NJ];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int j = 0; j < NJ; ++j) bias[q][j] = s_bias[q][wave * UPW + kgx + 4 * j];

  int probe_i = 0;
  // Probe steps live in SGPRs (a VGPR loaded in the loop would put a vmcnt(0) on every step).
  int probe_next = a.n_probe > 0 ? __builtin_amdgcn_readfirstlane(a.probe_steps[0]) : -1;
  auto write_probe = [&](int pi) {
    if (!row_ok) return;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int u = eu + 4 * j;
      if (u < a.H) {
        const size_t o = (((size_t)pi * a.L + layer) * a.B + grow) * a.H + u;
        a.probe_h[o] = (float)hcur[j];
        a.probe_c[o] = c[j];
      }
    }
  };

  uint64_t wv[NW] = {};  // poll results
  // The next layer's input: h_t of this slice's HS units x 16 rows, written a step later from
  // hbuf in 16-byte pieces, fragment-blocked (row block t * ntile + tile, column blocks of the
  // slice's units), by the first 2 HS threads.
  constexpr int kCopyThreads = HS * 16 / 8;
  const int copy_row = threadIdx.x & 15, copy_k8 = slice * (HS / 8) + (threadIdx.x >> 4) % (HS / 8);
  const int copy_src = copy_k8 * 16 + copy_row;  // f16x8 index of (row, units 8 copy_k8 ..) in hbuf
  f16x8* const copy_dst = last ? nullptr
                               : reinterpret_cast<f16x8*>(a.hout) + ((size_t)tile * (HP / 32) + (copy_k8 >> 2)) * 64 +
                                     (copy_k8 & 3) * 16 + copy_row;
  auto copy_out = [&](int t, const f16x8& v) { copy_dst[(size_t)t * a.ntile * (HP / 32) * 64] = v; };
  // The same copy inside the step loop (NJ = 2), as one 16-byte buffer store by every thread on every path:
  // a descriptor of step t's layer input (no bytes in the last layer), and threads past the copy
  // address it out of range, so their store is dropped.  The gather's wait for the ring poll then
  // leaves this store in flight (vmcnt(1)); with the store on some paths only, the compiler merged the
  // paths into a wait for every access in flight (vmcnt(0)), this store's completion included.
  const size_t copy_step = (size_t)a.ntile * (HP / 32) * 64;  // f16x8 per step of the layer input
  const unsigned copy_off =
      threadIdx.x < kCopyThreads
          ? (unsigned)((((size_t)tile * (HP / 32) + (copy_k8 >> 2)) * 64 + (copy_k8 & 3) * 16 + copy_row) * 16)
          : 0xFFFFFFF0u;
  auto copy_out_step = [&](int t, const f16x8& v) {
    const bool any = !last && t >= 0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        any ? reinterpret_cast<f16x8*>(a.hout) + (size_t)(any ? t : 0) * copy_step : nullptr, 0,
        any ? (int)(copy_step * 16) : 0, 0x00020000);
    typedef unsigned int u32x4c __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4c, v), rs, copy_off, 0, 0);
  };
  // One step: h_{t-1} in hbuf[t & 1] -> h_t in hbuf[(t + 1) & 1]; gp holds the input projection of
  // step t (X0: x_t) on entry and that of step t + 1 on return.  Returns false if a wait failed.
  // Step t + 1's projection is loaded first: it retires before this step's ring poll (loads retire
  // in order), about 2000 cycles later, so only stores are in flight when a step ends, on every
  // path (loop exits included), and the gate math never waits for a load.
  auto step = [&](int t, GV& gp) -> bool {
    GV gn = gload(t + 1);
    const f16x8* const hprev = hbuf[t & 1];
    f16x8* const hnext = hbuf[(t + 1) & 1];
    // The gate sums over all of K (X0: plus x_t W_ih^T) in two independent MFMA chains fed by one
    // 16-byte LDS read per K chunk: one chain per tile (NJ = 2), or the even and the odd K chunks of
    // the one tile (NJ = 1, summed before the gate math).
    // The accumulators start at bias + x_t W_ih^T (X0: at the bias), added here, where the second
    // wave of a SIMD waits for the matrix core anyway, rather than between the MFMAs and the gate math.
    f32x4 acc[2];
    if constexpr (NJ == 2) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[j][q] = X0 ? bias[q][j] : bias[q][j] + (float)gp[2 * q + j];
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[0][q] = X0 ? bias[q][0] : bias[q][0] + (float)gp[q];
      acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (X0) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wx[j], gp, acc[j], 0, 0, 0);
    }
    // The h fragments are read from LDS four K-chunks ahead of their MFMAs (one read in flight
    // per chunk would leave the matrix core waiting for LDS latency at every chunk).
    constexpr int kAhead = KCH < 4 ? KCH : 4;
    float cl0 = 0.f, hl0 = 0.f;  // unit eu's c and h of this step when chain 0 leads (kLead > 0)
    if constexpr (kLead > 0) {
      // Chain 0 (unit eu) runs kLead K-chunks ahead of chain 1 (unit eu + 4), and unit eu's cell
      // update is interleaved with chain 1's last kLead MFMAs instead of waiting for both chains:
      // the second wave of a SIMD, whose gate math is the step's critical path, starts it ~kLead
      // MFMAs earlier.  Fragment k is held from chain 0's MFMA to chain 1's.  Each chain sums in
      // the same order as before, so results are bit-identical (interleaved runs on two boxes: C4
      // 9.46-9.48 -> 9.38-9.41 ms on one, within its drift on the other; H512 B320 -0.5% to -1.5%;
      // I300 H256 -4% to -5% at a lead of 4; at H 256 a lead of 6 was 3.5% and one of 8, which leaves
      // no MFMA of chain 1 beside chain 0's, 1.5% slower; at H 128 a lead of 2 measured no change).
      constexpr int R = kAhead + kLead;
      f16x8 bq[R];
#pragma unroll
      for (int i = 0; i < kAhead; ++i) bq[i] = hprev[i * FV + lane];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int p = 0; p < KCH; ++p) {
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[p][0], bq[p % R], acc[0], 0, 0, 0);
        if (p >= kLead)
          acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[p - kLead][1], bq[(p - kLead) % R], acc[1], 0, 0, 0);
        if (p + kAhead < KCH) bq[(p + kAhead) % R] = hprev[(p + kAhead) * FV + lane];
        __builtin_amdgcn_sched_barrier(0);
      }
      // chain 1's last kLead MFMAs, each followed by a share of unit 0's cell update (~32 VALU
      // instructions; masks: 0x008 MFMA, 0x002 VALU)
#pragma unroll
      for (int p = KCH; p < KCH + kLead; ++p)
        acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[p - kLead][1], bq[(p - kLead) % R], acc[1], 0, 0, 0);
      {
        float cn = c[0], hn;
        lstm_cell(acc[0][0], acc[0][1], acc[0][2], acc[0][3], cn, hn);
        cl0 = cn;
        hl0 = hn;
        asm volatile("" : "+v"(cl0), "+v"(hl0));
      }
#pragma unroll
      for (int p = 0; p < kLead; ++p) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if constexpr (kLead >= 8)
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        else
          __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    } else {
      f16x8 bq[kAhead];
#pragma unroll
      for (int i = 0; i < kAhead; ++i) bq[i] = hprev[i * FV + lane];
#pragma unroll
      for (int kc = 0; kc < KCH; ++kc) {
        const f16x8 bv = bq[kc % kAhead];
        if (kc + kAhead < KCH) bq[kc % kAhead] = hprev[(kc + kAhead) * FV + lane];
        if constexpr (NJ == 2) {
          acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][0], bv, acc[0], 0, 0, 0);
          acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][1], bv, acc[1], 0, 0, 0);
        } else {
          acc[kc & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[kc][0], bv, acc[kc & 1], 0, 0, 0);
        }
      }
    }
    // h_{t-1} of this slice's units, 16 bytes per thread of the first 2 HS threads, stored below as
    // the next layer's input (hbuf[t & 1] is overwritten only in step t + 1).
    f16x8 hcp = {};
    if (!last && threadIdx.x < kCopyThreads) hcp = hprev[copy_src];

    // Gate math on the accumulators: gate q of unit eu + 4 j.
    const bool live = t < len;
    {
      float z[4][NJ];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < NJ; ++j) z[q][j] = NJ == 2 ? acc[j][q] : acc[0][q] + acc[1][q];
      float cn[NJ], hn[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (kLead > 0 && j == 0) {
          cn[0] = cl0;
          hn[0] = hl0;
          continue;
        }
        cn[j] = c[j];
        lstm_cell(z[0][j], z[1][j], z[2][j], z[3][j], cn[j], hn[j]);
      }
      // Both units' updates are computed on every lane and then selected: otherwise the compiler
      // puts each behind a branch on `live`, which serialises the two units' dependency chains.
      if constexpr (NJ == 2)
        asm volatile("" : "+v"(cn[0]), "+v"(cn[1]), "+v"(hn[0]), "+v"(hn[1]));
      else
        asm volatile("" : "+v"(cn[0]), "+v"(hn[0]));
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        c[j] = live ? cn[j] : c[j];
        hcur[j] = live ? (_Float16)hn[j] : hcur[j];
      }
    }

    // h_t: the tagged word for the sibling slices first, then the first poll of all words of step
    // t, and only then the stores and loads off the critical path (the next layer's input, the
    // output sequence, probes, the next step's input projection): loads and stores retire in issue
    // order, so the poll waits for nothing issued after it.
    // Tags of successive writes to a slot (steps t - 2, t) differ, and none is 0 (the cleared ring).
    const uint32_t want = xw_step_tag(t);
    const uint64_t want_bits = xw_tag_bits(want);  // its bits as the words carry them
    // This step's ring slot, uniform by construction: the compiler would otherwise keep its address
    // in VGPRs (it flows through the lane-conditional store) and put every poll in a waterfall loop.
    uint64_t* const slot = ring + (size_t)__builtin_amdgcn_readfirstlane(t & 1) * PW;
    // The word's two pairs: NJ = 2: (eu, eu + 1) and (eu + 4, eu + 5), this lane holding eu and
    // eu + 4, its partner lane + 16 (kgx + 1) eu + 1 and eu + 5.  NJ = 1: (eu, eu + 1) from this lane
    // and lane + 16, (eu + 2, eu + 3) from lanes + 32 and + 48 (the pair lane + 32 assembled).
    uint32_t pair_lo, pair_hi;
    {
      uint32_t bits = (uint32_t)__builtin_bit_cast(uint16_t, hcur[0]);
      if constexpr (NJ == 2) bits |= (uint32_t)__builtin_bit_cast(uint16_t, hcur[1]) << 16;
      const uint32_t mine = xw_enc_pair(bits);
      const uint32_t other = (uint32_t)__builtin_amdgcn_ds_swizzle((int)mine, 0x401F);  // lane ^ 16
      pair_lo = __builtin_amdgcn_perm(other, mine, 0x05040100u);
      if constexpr (NJ == 2)
        pair_hi = __builtin_amdgcn_perm(other, mine, 0x07060302u);
      else
        pair_hi = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane + 32) & 63) << 2, (int)pair_lo);
      const uint64_t word = ((uint64_t)pair_lo | ((uint64_t)pair_hi << 32)) | want_bits;
      if (writer) {
        if (l2)
          __hip_atomic_store(slot + pwoff, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else
          __hip_atomic_store(slot + pwoff, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // The poll reads two adjacent words of a sibling per 16-byte buffer load with cache policy sc1 (what
    // agent-scope relaxed atomics compile to): a descriptor of the ring slot in SGPRs (word 3
    // 0x00020000: DATA_FORMAT = 32 bit, which untyped buffer accesses need on CDNA), the thread's
    // byte offset in one VGPR, the block offset as the scalar offset, every offset inside the slot.
    // Each word is written by one aligned 8-byte atomic store and lies inside one aligned 16-byte
    // load, so it is read whole; its own tag validates it (the two words of a load may come from
    // different steps, and a load is repeated until both are current).  Half the load
    // instructions of 8-byte atomic loads: C4 21.5 -> 20.0 ms.
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(slot, 0, PW * 8, 0x00020000);
    auto pload = [&](int p) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, (unsigned)q_in * 16u, sib(p) * HS * 32, 16);
      wv[2 * p] = (uint64_t)v[0] | ((uint64_t)v[1] << 32);
      wv[2 * p + 1] = (uint64_t)v[2] | ((uint64_t)v[3] << 32);
    };
    // A first poll that finds a sibling's word not yet written costs a round trip (~800 cycles
    // under load), so every wave waits before polling: the first wave of each SIMD (waves 0-3)
    // finishes its cell updates ~500 cycles before the second (the matrix core serves the older
    // wave first) and waits longer.  The branch is on a wave-uniform value: s_sleep ignores the exec
    // mask, so under a lane-masked branch every wave would sleep.  Only the poll is delayed.  The
    // delays (units of 64 cycles) are per padded H, from interleaved runs on one box each: 14 / 6
    // had been chosen at C4 when the layer-input store still held up the poll's wait (no wait 12.23
    // ms, 512 cycles for all waves 11.48-11.92, 14 / 6 11.27-11.85); after it, H512 B320 8.36 ->
    // 8.02 ms and B448 9.13 -> 8.95 ms at 10 / 4 (8 / 2: 7.98 and 9.02), I300 H256 7.55 -> 7.17 ms at
    // 8 / 2 (10 / 4: 7.24), H1024 41.9 -> 41.45 ms at 12 / 2 (10 / 4: 41.65); C4 within the noise
    // of the box (-1.4% to -1.8% at 10 / 4 on three others).
    constexpr int kPollSleepFirst = HP >= 1024 ? 12 : HP == 512 ? 10 : 8;
    constexpr int kPollSleepSecond = HP == 512 ? 4 : 2;
    if (__builtin_amdgcn_readfirstlane(wave) < 4)
      __builtin_amdgcn_s_sleep(kPollSleepFirst);
    else
      __builtin_amdgcn_s_sleep(kPollSleepSecond);
#pragma unroll
    for (int p = 0; p < NL; ++p)
      if (has_ld(p)) pload(p);
    // This slice's own pairs of h_t, from the lanes that send them (nobody reads hbuf[(t + 1) & 1]
    // in step t).
    if (writer) {
      uint32_t* own32 = reinterpret_cast<uint32_t*>(hnext);
      own32[own_dst] = xw_dec_pair(pair_lo);
      own32[own_dst + (NJ == 2 ? 2 : 1)] = xw_dec_pair(pair_hi);
    }
    if constexpr (NJ == 2) {
      copy_out_step(t - 1, hcp);
    } else if (!last && threadIdx.x < kCopyThreads && t > 0) {
      copy_out(t - 1, hcp);  // (at padded H 1024 the store on every path measured 1.2% slower)
    }
    if (last && a.out_seq && row_ok) {
      _Float16* dst = a.out_seq + ((size_t)grow * a.T + t) * a.H + eu;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (eu + 4 * j < a.H) dst[4 * j] = live ? hcur[j] : (_Float16)0.0f;
    }
    if (t + 1 == probe_next) {
      write_probe(probe_i);
      ++probe_i;
      probe_next = probe_i < a.n_probe ? __builtin_amdgcn_readfirstlane(a.probe_steps[probe_i]) : -1;
    }

    // Gather h_t of every slice: re-poll the words whose tag is not step t's yet (bounded wait).
    uint64_t t0 = 0;
    for (int spin = 0;; ++spin) {
      bool ready = true;
#pragma unroll
      for (int r = 0; r < NW; ++r) ready = ready & (!has_ld(r >> 1) || xw_tag_is(wv[r], want_bits));
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
      for (int p = 0; p < NL; ++p)
        if (has_ld(p) && !(xw_tag_is(wv[2 * p], want_bits) & xw_tag_is(wv[2 * p + 1], want_bits))) pload(p);
    }
    // gn's load was issued before this step's poll, so it has completed (loads retire in order);
    // the empty asm tells the compiler, which would otherwise count the copy below as a read of a
    // load in flight.
    // Failure injection for tests (plh_inject_wait_failure): workgroup 0 treats this step's wait as
    // timed out; its siblings then find the status word set while they wait for its next words.
    if (t == a.fail_step && blockIdx.x == 0) {
      s_fail = 1;
      if (threadIdx.x == 0)
        __hip_atomic_fetch_or(a.status, PLH_STATUS_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("" : "+v"(gn));
    gp = gn;
#pragma unroll
    for (int k = 0; k < NL; ++k)
      if (has_ld(k)) {
        // NJ = 2: words 2 k (units +0, +1 | +4, +5) and 2 k + 1 (+2, +3 | +6, +7) of one row;
        // NJ = 1: words 2 k (units +0, +1 | +2, +3) and 2 k + 1 (+4, +5 | +6, +7).
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        const uint32_t a0 = xw_dec_pair((uint32_t)wv[2 * k]), a1 = xw_dec_pair((uint32_t)(wv[2 * k] >> 32));
        const uint32_t b0 = xw_dec_pair((uint32_t)wv[2 * k + 1]), b1 = xw_dec_pair((uint32_t)(wv[2 * k + 1] >> 32));
        const u32x4 v = NJ == 2 ? u32x4{a0, b0, a1, b1} : u32x4{a0, a1, b0, b1};
        hnext[gdst16(k)] = __builtin_bit_cast(f16x8, v);
      }
    lds_barrier();
    return __builtin_amdgcn_readfirstlane(s_fail) == 0;
  };

  GV gp = {};
  if (Tt > 0) gp = gload(0);
  // Nothing in flight at the loop entry, so the first gate math waits for no load.
  wait_vmem_all();
  bool ok = __builtin_amdgcn_readfirstlane(s_fail) == 0;
  for (int t = 0; ok && t < Tt; ++t) ok = step(t, gp);
  // Rows of length 0 keep their h0, which the packed exchange may not carry intact: restore their
  // h in hbuf before it is read as a result (the last copy-out, the head).
  if (ok && a.lengths && Tt > 0) {
    for (int idx = threadIdx.x; idx < KCH * FV; idx += NT) {
      const int kc = idx / FV, l = idx % FV;
      const int gr = a.row0 + tile * 16 + (l & 15);
      if (gr >= a.row_end || a.lengths[gr] > 0) continue;
      const int k0 = kc * 32 + (l >> 4) * 8;
      f16x8 v = {};
      if (a.h0) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (k0 + j < a.H) v[j] = a.h0[((size_t)layer * a.B + gr) * a.H + k0 + j];
      }
      hbuf[Tt & 1][idx] = v;
    }
    __syncthreads();
  }
  // The last step's h (in hbuf[Tt & 1] after its gather) as the next layer's input.
  if (ok && !last && Tt > 0 && threadIdx.x < kCopyThreads) copy_out(Tt - 1, hbuf[Tt & 1][copy_src]);

  if (!ok) {
    // A wait failed, here or in an earlier layer's launch (the status word records it): poison every
    // output of this workgroup (states, probes, output sequence, head) and leave.
    if (row_ok) poison_lane_outputs(a, layer, grow, eu, NJ, last, 4);
    if (last && slice == 0 && a.out) {
      for (int idx = threadIdx.x; idx < 16 * a.O; idx += NT) {
        const int gr = a.row0 + tile * 16 + idx / a.O;
        if (gr < a.row_end) a.out[(size_t)gr * a.O + idx % a.O] = (_Float16)__builtin_nanf("");
      }
    }
    return;
  }

  // Steps past the tile's longest row were never visited: their output sequence is zero.
  if (last && a.out_seq && row_ok) {
    for (int t = Tt; t < a.T; ++t) {
      _Float16* dst = a.out_seq + ((size_t)grow * a.T + t) * a.H + eu;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (eu + 4 * j < a.H) dst[4 * j] = (_Float16)0.0f;
    }
  }
  // ... and the next layer's input there is the frozen state (its rows are frozen as well).
  while (probe_i < a.n_probe) {
    write_probe(probe_i);
    ++probe_i;
  }
  if (row_ok) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int u = eu + 4 * j;
      if (u < a.H) {
        const size_t si = ((size_t)layer * a.B + grow) * a.H + u;
        if (a.h_n) a.h_n[si] = hcur[j];
        if (a.c_n) a.c_n[si] = (_Float16)c[j];
      }
    }
  }
  // Linear head (last layer, first slice) on the full final h held in hbuf[Tt & 1].
  if (last && slice == 0 && a.out) {
    for (int idx = threadIdx.x; idx < 16 * a.O; idx += NT) {
      const int rr = idx / a.O, o = idx % a.O;
      const int gr = a.row0 + tile * 16 + rr;
      if (gr >= a.row_end) continue;
      const _Float16* hf = reinterpret_cast<const _Float16*>(hbuf[Tt & 1]);
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

inline unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per); }

template <int HP>
hipError_t pack_rec_layer_hp(int H, const _Float16* w_hh, _Float16* dst, hipStream_t s) {
  const size_t n = (size_t)4 * HP * HP;
  hipLaunchKernelGGL(pack_rec_kernel<HP>, blocks_for(n, 256), 256, 0, s, w_hh, H, dst);
  return hipGetLastError();
}

template <int HP>
hipError_t pack_rec_wx0_hp(int H, int I, const _Float16* w_ih0, _Float16* dst, hipStream_t s) {
  const size_t n = (size_t)HP * 128;
  hipLaunchKernelGGL(pack_rec_wx0_kernel<HP>, blocks_for(n, 256), 256, 0, s, w_ih0, H, I, dst);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_pack_rec_layer(const Geometry& g, int layer, const _Float16* w_hh, _Float16* wpack, hipStream_t s) {
  _Float16* dst = wpack + (size_t)layer * 4 * g.HP * g.HP;
  switch (g.HP) {
    case 128: return pack_rec_layer_hp<128>(g.H, w_hh, dst, s);
    case 256: return pack_rec_layer_hp<256>(g.H, w_hh, dst, s);
    case 512: return pack_rec_layer_hp<512>(g.H, w_hh, dst, s);
    case 1024: return pack_rec_layer_hp<1024>(g.H, w_hh, dst, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pack_rec_wih(const Geometry& g, const _Float16* w_ih, int K, int Kp, _Float16* dst, hipStream_t s) {
  const size_t n = (size_t)4 * g.HP * Kp;
  hipLaunchKernelGGL(pack_rec_wih_kernel, blocks_for(n, 256), 256, 0, s, w_ih, g.H, g.HP, K, Kp, dst);
  return hipGetLastError();
}

hipError_t launch_pack_rec_wx0(const Geometry& g, const _Float16* w_ih0, _Float16* dst, hipStream_t s) {
  if (g.I > 32) return hipErrorInvalidValue;
  switch (g.HP) {
    case 512: return pack_rec_wx0_hp<512>(g.H, g.I, w_ih0, dst, s);
    case 1024: return pack_rec_wx0_hp<1024>(g.H, g.I, w_ih0, dst, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rec_input(const Geometry& g, const ForwardArgs& a, _Float16* xs0, int ld, hipStream_t s) {
  const size_t n = (size_t)a.T * a.rows_pad * g.kp0;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(rec_input_kernel, blocks_for(n, 256), 256, 0, s, a.x, a.T, g.I, a.row0, a.row_end, a.rows_pad,
                     ld, g.kp0, xs0);
  return hipGetLastError();
}

const void* rec_kernel(int HP, bool x0) {
  switch (HP) {
    case 128: return x0 ? nullptr : reinterpret_cast<const void*>(&lstm_rec_kernel<128, false>);
    case 256: return x0 ? nullptr : reinterpret_cast<const void*>(&lstm_rec_kernel<256, false>);
    case 512:
      return x0 ? reinterpret_cast<const void*>(&lstm_rec_kernel<512, true>)
                : reinterpret_cast<const void*>(&lstm_rec_kernel<512, false>);
    case 1024:
      return x0 ? reinterpret_cast<const void*>(&lstm_rec_kernel<1024, true>)
                : reinterpret_cast<const void*>(&lstm_rec_kernel<1024, false>);
    default: return nullptr;
  }
}

}  // namespace plh
