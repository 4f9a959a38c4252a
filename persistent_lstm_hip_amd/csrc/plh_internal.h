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
  int HP;      // padded hidden size: 32, 64, 128 (one workgroup per layer and tile), 256, 512 (sliced)
               // or 1024 (layer-sequential only); 128 at least when I > HP
  int slices;  // workgroups per (layer, tile): 1, 4 (HP = 256), 16 (HP = 512); on the layer-sequential
               // path Rec<HP>::kS (2, 4, 8, 32)
  int wave_ok;  // the all-layers kernels serve this geometry (HP <= 512 and I <= HP)
  int rec_ok;  // the layer-sequential path serves it (HP >= 512, or I > HP): its weights are packed too
  int rec;     // this forward runs layer by layer: input projection as a GEMM, recurrent kernel
               // holding W_hh alone (make_geometry leaves 0; as_layer_sequential sets it)
  int max_wg_tiles;  // 16-row tiles a sliced workgroup can carry (2 at HP = 256, software-pipelined)
  int waves;   // waves per workgroup: HP / 16 (one per 16 hidden units) or 8 when sliced
  int kci;     // input-part K chunks of 32 for layers >= 1 (= HP / 32)
  int kc;      // K chunks of [W_ih | W_hh] per gate row (= 2 * kci)
  int g_in0;   // 8-wide K groups of x per step that layer 0 reads (= ceil(I / 8) <= 4 * kci); on the
               // layer-sequential path with rec_x0, 4 (one zero-padded K chunk of 32)
  int rec_x0;  // layer-sequential path: layer 0's input projection (I <= 32) is computed inside the
               // recurrent kernel (one MFMA K chunk); otherwise by the projection GEMM like the others
  int kp0, kp;  // K of the projection GEMM, padded to a multiple of 128: layer 0 (0 with rec_x0), layers >= 1
};
// The layer-sequential path's padded hidden sizes and the largest hidden size served.
constexpr int kMaxHidden = 1024;

// u32 words per (layer, tile) counter: the sliced kernels' counters each take a 128-byte line of
// their own (their workgroups read and update them every few steps, and counters sharing a line
// serialise those accesses); the wavefront kernels' are adjacent.
constexpr int kSlicedCounterStride = 32;
inline int counter_stride(const Geometry& g) { return g.slices > 1 && !g.rec ? kSlicedCounterStride : 1; }

// Fills *g; returns false (with the reason) for geometries the kernels do not implement.
bool make_geometry(int I, int H, int L, int O, Geometry* g, std::string* why);
// g (rec_ok) switched to the layer-sequential path.
Geometry as_layer_sequential(const Geometry& g);

// Byte offsets of the packed-weight blob (all 256-byte aligned).
struct PackedLayout {
  size_t wpack;  // f16 MFMA A fragments of every lane: [L][waves][kc][4 gates][64 lanes][8], or when
                 // sliced [L][slices][8 waves][2 KCH chunks][NJ tiles][64 lanes][8] (Sliced<HP>)
  size_t bias;   // f32 [L][4][HP]: b_ih + b_hh
  size_t wlin;   // f32 [O][HP]
  size_t blin;   // f32 [O]
  size_t wrec;   // rec_ok: f16 W_hh fragments of the layer-sequential kernel, [L][S slices][8 waves][HP / 32
                 // chunks][NJ tiles][64 lanes][8] (Rec<HP>)
  size_t wih;    // rec_ok: f16 W_ih of every layer the projection GEMM computes, as its W operand:
                 // [4 HP][kp0] (layer 0, unless rec_x0), then [4 HP][kp] per layer >= 1; rows permuted to the
                 // recurrent kernel's lane order, K zero-padded
  size_t wx0;    // rec_ok with rec_x0: f16 MFMA A fragments of W_ih of layer 0 for the recurrent kernel,
                 // [S slices][8 waves][NJ tiles][64 lanes][8] (HP x 128 halfs)
  size_t total;
};
PackedLayout packed_layout(const Geometry& g);

// Workspace of one persistent launch (reused by successive batch chunks); R = rows per tile:
//   status   u32                                   PLH_STATUS_* bits
//   counters u32 [L][ntile][counter_stride]       progress published per (layer, tile)
//   xp       f16x8 [ntile][T][g_in0][R]            x in B-fragment order (layer 0 input): group g
//                                                  holds k = 8g .. 8g+7, the first g_in0 * R
//                                                  entries of a step's fragment blocks
//   hseq     f16x8 [L-1][ntile][T][kci][4][R]      h of layers 0..L-2 in B-fragment order
//   xring    u64 [L][ntile][2][HP * 8]             sliced geometries only: per-step exchange of h
//                                                  among the slices of a (layer, tile), tagged words;
//            then u32 [L][ntile][16]               the XCD id (+1) of every slice of a group
// Layer-sequential geometries (one layer per launch) use instead of xp and hseq:
//   gates    f16 [T * rows][4 HP] fragment-blocked one layer's input projection x_t W_ih^T, columns
//                                                  in the recurrent kernel's lane order
//   xs       f16 [2][T * rows][HP] fragment-blocked layer inputs/outputs, alternating (x in slot 0
//                                                  when layer 0's projection is a GEMM and kp0 <= HP)
//   xin      f16 [T * rows][kp0]   fragment-blocked x, when layer 0's projection is a GEMM with
//                                                  kp0 > HP (input size above the padded H)
// (fragment-blocked: see blocked_index; one 1 KB block per 16 rows x 32 columns)
//   xp       f16x8 [ntile][T][4][16]               with rec_x0: x in B-fragment order, K zero-padded
//                                                  to 32 (layer 0's in-kernel projection)
// and an xring of one layer, followed by u32 [ntile][8]: the XCD id of each slice (+1), zeroed with
// the ring before each launch.
struct WorkspaceLayout {
  size_t status, counters, xp, hseq, xring, gates, xs, xin, total;
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
  uint32_t* counters;           // [L][ntile][counter_stride] progress published per (layer, tile)
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
  int fail_step;                // failure injection (plh_inject_wait_failure): the layer-sequential kernel's
                                // workgroup 0 fails its wait at this step; -1: never
  int wg_tiles;                 // sliced kernels: 16-row tiles per workgroup (1 or 2); ntile is a multiple
  // layer-sequential kernel (one layer per launch):
  int layer;                    // the layer this launch runs
  int ntile_grid;               // tiles the launch's grid covers (>= ntile: a multiple of 8 where that fits,
                                // so that every tile's slices share an XCD); the extra ones exit at once
  int groups_grid;              // sliced kernels: (layer, tile group) groups the grid covers (>= L ntile /
                                // wg_tiles, rounded up to 8 the same way; 0: exactly those)
  const _Float16* gates;        // [T * rows_pad][4 HP] blocked: input projection of that layer (no bias), lane order
  _Float16* hout;               // [T * rows_pad][HP] blocked: its h sequence, the next layer's input (null: last layer)
  const _Float16* wx0;          // rec_x0, layer 0: W_ih fragments of the in-kernel projection (x from xp)
};

hipError_t launch_pack_layer(const Geometry& g, int layer, const _Float16* w_ih, const _Float16* w_hh,
                             _Float16* wpack, hipStream_t s);
hipError_t launch_pack_bias(const Geometry& g, int layer, const _Float16* b_ih, const _Float16* b_hh,
                            float* bias, hipStream_t s);
hipError_t launch_pack_linear(const Geometry& g, const _Float16* w, const _Float16* b, float* wlin,
                              float* blin, hipStream_t s);
// One launch before each persistent launch: packs this launch's x into xp (g0 8-wide K groups per
// row and step, zero past I) and clears the status word (if `status`), the counters and ring_words
// u64 words of the exchange ring.
hipError_t launch_forward_prologue(const Geometry& g, const ForwardArgs& a, uint32_t* status, int g0,
                                   size_t ring_words, hipStream_t s);
hipError_t launch_zero_u32(uint32_t* p, size_t n, hipStream_t s);
hipError_t launch_repeat_first_row(const _Float16* in, _Float16* out, int rows, int cols, hipStream_t s);

// Persistent kernels (device function pointers for hipLaunchKernel), nullptr if no variant
// exists: the wavefront kernel for padded H <= 128 and 8- or 16-row tiles (plh_wavefront.hip), the
// sliced kernel for padded H 256 / 512 with 1 or 2 tiles per workgroup (plh_sliced.hip).
const void* wavefront_kernel(int HP, int tile_rows, bool ragged);
const void* sliced_kernel(int HP, int wg_tiles);

// Co-resident workgroups of the persistent kernel on the current device (0 with *err set on error).
int recurrent_capacity(const Geometry& g, int tile_rows, hipError_t* err);
hipError_t launch_recurrent(const Geometry& g, const ForwardArgs& a, hipStream_t s);

// Layer-sequential path (plh_rec.hip): W_hh fragments of one layer, x of a launch's rows into the
// first GEMM's input (blocked [T * rows_pad][ld], zero past the launch's rows and past I up to kp0),
// and the recurrent kernel of a.layer (x0: with layer 0's in-kernel input projection).
hipError_t launch_pack_rec_layer(const Geometry& g, int layer, const _Float16* w_hh, _Float16* wpack, hipStream_t s);
hipError_t launch_rec_input(const Geometry& g, const ForwardArgs& a, _Float16* xs0, int ld, hipStream_t s);
// W_ih ([4H][K]) of one layer as the projection GEMM's W operand ([4 HP][Kp], lane-ordered rows,
// zero columns K..Kp-1).
hipError_t launch_pack_rec_wih(const Geometry& g, const _Float16* w_ih, int K, int Kp, _Float16* dst, hipStream_t s);
// W_ih of layer 0 (I <= 32) as the recurrent kernel's MFMA A fragments (PackedLayout::wx0).
hipError_t launch_pack_rec_wx0(const Geometry& g, const _Float16* w_ih0, _Float16* dst, hipStream_t s);
const void* rec_kernel(int HP, bool x0);

// Time-parallel input projection (plh_gemm.hip): C[m][n] = sum_k X[m][k] W[n][k] for m < M, n < N,
// fp16 operands and result, fp32 accumulation.  Row-major X [M][ldx], W [N][K], C [M][ldc], or with
// `blocked` X and C in fragment-blocked order, [M / 16][ld / 32][64 lanes][8] (block (mb, g), lane l:
// row 16 mb + l % 16, columns 32 g + 8 (l / 16) + 0..7).  K % 128 == 0, K <= kGemmMaxKTotal,
// N % 128 == 0, ldx >= K and ldc >= N multiples of 8 (blocked: of 32, M % 16 == 0), 16-byte aligned
// pointers (gemm_shape_ok).  A persistent launch of about one workgroup per CU.
constexpr int kGemmMaxKTotal = 1 << 16;
bool gemm_shape_ok(long long M, int N, int K, long long ldx, long long ldc, bool blocked);
hipError_t launch_proj_gemm(const _Float16* X, long long ldx, const _Float16* W, int K, _Float16* C, long long ldc,
                            long long M, int N, bool blocked, int cus, hipStream_t s);
// Offset (in halfs) of element (row r, column k) of a fragment-blocked [rows / 16][ld / 32][64][8] matrix.
__host__ __device__ inline size_t blocked_index(size_t r, int k, int ld) {
  return (((r >> 4) * (size_t)(ld >> 5) + (k >> 5)) * 64 + ((k >> 3) & 3) * 16 + (r & 15)) * 8 + (k & 7);
}
double proj_gemm_flops(long long M, int N, int K);

// MFMA rate probe (plh_probe.hip): `blocks` workgroups of 16 waves (one per CU), each wave issuing
// iters x 8 independent v_mfma_f32_16x16x32_f16; out holds blocks x 1024 floats, clk blocks x 2
// (shader cycles, 100 MHz ticks of the loop).  mfma_probe_flops: the FLOPs of one launch.
hipError_t launch_mfma_probe(int blocks, int iters, float* out, unsigned long long* clk, hipStream_t s);
double mfma_probe_flops(int blocks, int iters);

}  // namespace plh
