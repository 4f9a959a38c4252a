// plh_internal.h -- declarations shared by the kernel sources (plh_wavefront.hip, plh_sliced.hip,
// plh_pack.hip, plh_launch.hip, plh_probe.hip) and the C ABI (plh_capi.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace plh {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// Geometry of one model as the kernels see it.  H is padded to HP (a bucket the kernel is
// instantiated for); padded hidden units carry zero weights and zero bias, so their gates are
// i = f = o = 0.5, g = 0 and their c and h stay exactly 0: padding never changes real outputs.
struct Geometry {
  int I, H, L, O;
  int HP;      // padded hidden size: 32, 64, 128 (one workgroup per layer and tile), 256 (sliced) or
               // 512 (layer-sequential)
  int slices;  // workgroups per (layer, tile): 1, 4 (HP = 256), 16 (HP = 512) or 8 (layer-sequential)
  int rec_ok;  // HP = 512: the layer-sequential path exists (its weights are packed too)
  int rec;     // this forward runs layer by layer: input projection as a GEMM, recurrent kernel
               // holding W_hh alone (make_geometry leaves 0; as_layer_sequential sets it)
  int max_wg_tiles;  // 16-row tiles a sliced workgroup can carry (2 at HP = 256, software-pipelined)
  int waves;   // waves per workgroup: HP / 16 (one per 16 hidden units) or 8 when sliced
  int kci;     // input-part K chunks of 32 for layers >= 1 (= HP / 32)
  int kc;      // K chunks of [W_ih | W_hh] per gate row (= 2 * kci)
  int g_in0;   // 8-wide K groups of x per step that layer 0 reads (= ceil(I / 8) <= 4 * kci)
};

// Fills *g; returns false (with the reason) for geometries the kernels do not implement.
bool make_geometry(int I, int H, int L, int O, Geometry* g, std::string* why);
// g (rec_ok) switched to the layer-sequential path.
Geometry as_layer_sequential(const Geometry& g);

// Byte offsets of the packed-weight blob (all 256-byte aligned).
struct PackedLayout {
  size_t wpack;  // f16 MFMA A fragments of every lane: [L][waves][kc][4 gates][64 lanes][8], or when
                 // sliced [L][slices][8 waves][8 chunks][4 gates][64 lanes][8]
  size_t bias;   // f32 [L][4][HP]: b_ih + b_hh
  size_t wlin;   // f32 [O][HP]
  size_t blin;   // f32 [O]
  size_t wrec;   // rec_ok: f16 W_hh fragments of the layer-sequential kernel, [L][8 slices][8 waves][8
                 // chunks][4 gates][64 lanes][8]
  size_t wih;    // rec_ok: f16 W_ih of every layer as the projection GEMM's A operand, [4 HP][I], then
                 // [4 HP][H] per layer: rows permuted to the kernel's lane order
  size_t total;
};
PackedLayout packed_layout(const Geometry& g);

// Workspace of one persistent launch (reused by successive batch chunks); R = rows per tile:
//   status   u32                                   PLH_STATUS_* bits
//   counters u32 [L][ntile]                        steps published per (layer, tile)
//   xp       f16x8 [ntile][T][g_in0][R]            x in B-fragment order (layer 0 input): group g
//                                                  holds k = 8g .. 8g+7, the first g_in0 * R
//                                                  entries of a step's fragment blocks
//   hseq     f16x8 [L-1][ntile][T][kci][4][R]      h of layers 0..L-2 in B-fragment order
//   xring    u64 [L][ntile][2][HP * 8]             sliced geometries only: per-step exchange of h
//                                                  among the slices of a (layer, tile), tagged words
// Layer-sequential geometries (one layer per launch) use instead of xp and hseq:
//   gates    f16 [T][rows][4 HP]                   one layer's input projection x_t W_ih^T, columns
//                                                  in the recurrent kernel's lane order
//   xs       f16 [2][T][rows][HP]                  layer inputs/outputs, alternating (x in slot 0)
// and an xring of one layer.
struct WorkspaceLayout {
  size_t status, counters, xp, hseq, xring, gates, xs, total;
  size_t xring_words;  // u64 words of xring (0 unless sliced)
  int chunk_rows;  // batch rows per persistent launch (co-residency bound), multiple of tile_rows
  int tile_rows;   // batch rows per workgroup: 8 or 16
};
WorkspaceLayout workspace_layout(const Geometry& g, int seq_len, int chunk_rows, int tile_rows);

struct ForwardArgs {
  const _Float16* x;            // [B, T, I]
  const int32_t* lengths;       // [B] or null
  const _Float16* wpack;        // packed blob sections
  const float* bias;
  const float* wlin;
  const float* blin;
  f16x8_t* xp;                  // packed x, see WorkspaceLayout
  f16x8_t* hseq;                // inter-layer hand-off, see WorkspaceLayout
  uint64_t* xring;              // sliced kernels: tagged h exchange ring, zeroed before each launch
  uint32_t* counters;           // [L][ntile] steps published per (layer, tile)
  uint32_t* status;             // PLH_STATUS_* bits
  const _Float16* h0;           // [L, B, H] or null
  const _Float16* c0;
  _Float16* out;                // [B, O] or null
  _Float16* out_seq;            // [B, T, H] or null
  _Float16* h_n;                // [L, B, H] or null
  _Float16* c_n;
  const int32_t* probe_steps;   // [n_probe], strictly increasing
  float* probe_h;               // [n_probe, L, B, H]
  float* probe_c;
  int n_probe;
  int B, T, I, H, L, O;
  int row0, row_end;            // batch rows [row0, row_end) handled by this launch
  int rows_pad, ntile;          // rows_pad = tile_rows * ntile
  int tile_rows;                // batch rows per workgroup: 8 or 16
  int g_in0;                    // 8-wide K groups of x per step in xp
  int xcd_map;                  // 1: keep a tile's layer chain on one XCD
  uint64_t wait_ticks;          // bound on one inter-workgroup wait, in s_memrealtime ticks (100 MHz)
  int wg_tiles;                 // sliced kernels: 16-row tiles per workgroup (1 or 2); ntile is a multiple
  // layer-sequential kernel (one layer per launch):
  int layer;                    // the layer this launch runs
  const _Float16* gates;        // [T][rows_pad][4 HP] input projection of that layer (no bias), lane order
  _Float16* hout;               // [T][rows_pad][HP] its h sequence, the next layer's input (null: last layer)
};

hipError_t launch_pack_layer(const Geometry& g, int layer, const _Float16* w_ih, const _Float16* w_hh,
                             _Float16* wpack, hipStream_t s);
hipError_t launch_pack_bias(const Geometry& g, int layer, const _Float16* b_ih, const _Float16* b_hh,
                            float* bias, hipStream_t s);
hipError_t launch_pack_linear(const Geometry& g, const _Float16* w, const _Float16* b, float* wlin,
                              float* blin, hipStream_t s);
// One launch before each persistent launch: packs this launch's x into xp and clears the status
// word (if `status`), the counters and (sliced) the exchange ring.
hipError_t launch_forward_prologue(const Geometry& g, const ForwardArgs& a, uint32_t* status, hipStream_t s);
hipError_t launch_zero_u32(uint32_t* p, size_t n, hipStream_t s);
hipError_t launch_repeat_first_row(const _Float16* in, _Float16* out, int rows, int cols, hipStream_t s);

// Persistent kernels (device function pointers for hipLaunchCooperativeKernel), nullptr if no variant
// exists: the wavefront kernel for padded H <= 128 and 8- or 16-row tiles (plh_wavefront.hip), the
// sliced kernel for padded H 256 / 512 with 1 or 2 tiles per workgroup (plh_sliced.hip).
const void* wavefront_kernel(int HP, int tile_rows, bool ragged);
const void* sliced_kernel(int HP, int wg_tiles);

// Co-resident workgroups of the persistent kernel on the current device (0 with *err set on error).
int recurrent_capacity(const Geometry& g, int tile_rows, hipError_t* err);
hipError_t launch_recurrent(const Geometry& g, const ForwardArgs& a, hipStream_t s);

// Layer-sequential path (plh_rec.hip): W_hh fragments of one layer, x of a launch's rows into
// xs slot 0 ([T][rows_pad][HP], zero past the launch's rows), and the recurrent kernel of a.layer.
hipError_t launch_pack_rec_layer(const Geometry& g, int layer, const _Float16* w_hh, _Float16* wpack, hipStream_t s);
hipError_t launch_rec_input(const Geometry& g, const ForwardArgs& a, _Float16* xs0, hipStream_t s);
// W_ih ([4H][K]) of one layer as the projection GEMM's A operand ([4 HP][K], lane-ordered rows).
hipError_t launch_pack_rec_wih(const Geometry& g, const _Float16* w_ih, int K, _Float16* dst, hipStream_t s);
const void* rec_kernel(int HP);

// MFMA rate probe (plh_probe.hip): `blocks` workgroups of 16 waves (one per CU), each wave issuing
// iters x 8 independent v_mfma_f32_16x16x32_f16; out holds blocks x 1024 floats, clk blocks x 2
// (shader cycles, 100 MHz ticks of the loop).  mfma_probe_flops: the FLOPs of one launch.
hipError_t launch_mfma_probe(int blocks, int iters, float* out, unsigned long long* clk, hipStream_t s);
double mfma_probe_flops(int blocks, int iters);

}  // namespace plh
