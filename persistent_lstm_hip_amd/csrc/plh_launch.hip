// plh_launch.hip -- host side of the kernels: geometry rules, buffer layouts, kernel choice,
// occupancy and the launch of the persistent recurrence.
#include <algorithm>

#include "plh_device.h"

namespace plh {

bool make_geometry(int I, int H, int L, int O, Geometry* g, std::string* why) {
  if (I <= 0 || H <= 0 || L <= 0 || O < 0) {
    *why = "input_size, hidden_size and num_layers must be positive and output_size non-negative";
    return false;
  }
  if (H > kMaxHidden) {
    *why = "hidden_size > 1024 is not implemented by the persistent kernels";
    return false;
  }
  if ((long long)I > (long long)kGemmMaxKTotal) {
    *why = "input_size > 65536 is not implemented";
    return false;
  }
  if (L > 64 || O > 4096) {
    *why = "num_layers > 64 or output_size > 4096 is not implemented";
    return false;
  }
  int HP = H <= 32 ? 32 : H <= 64 ? 64 : H <= 128 ? 128 : H <= 256 ? 256 : H <= 512 ? 512 : 1024;
  // An input wider than the padded hidden size does not fit the all-layers kernels' resident input
  // part: such a model runs layer by layer (its layer-0 projection a GEMM over any K), whose kernels
  // start at padded H 128 (the extra padded units stay exactly zero).
  if (I > HP && HP < 128) HP = 128;
  g->I = I;
  g->H = H;
  g->L = L;
  g->O = O;
  g->HP = HP;
  g->wave_ok = (HP <= 512 && I <= HP) ? 1 : 0;
  g->rec_ok = (HP >= 512 || I > HP) ? 1 : 0;
  g->rec = 0;
  g->slices = HP == 256 ? Sliced<256>::kS : HP == 512 ? Sliced<512>::kS : 1;
  g->max_wg_tiles = HP == 256 ? 2 : 1;
  g->waves = g->slices > 1 ? 8 : HP / 16;
  g->kci = HP / 32;
  g->kc = 2 * g->kci;
  g->g_in0 = (I + 7) / 8;
  // Layer 0's projection inside the recurrent kernel: one MFMA K chunk of x (I <= 32), at H 512 / 1024.
  g->rec_x0 = (g->rec_ok && HP >= 512 && I <= 32) ? 1 : 0;
  g->kp0 = g->rec_x0 ? 0 : (I + 127) / 128 * 128;
  g->kp = (H + 127) / 128 * 128;
  return true;
}

Geometry as_layer_sequential(const Geometry& g) {
  Geometry r = g;
  r.rec = 1;
  r.slices = rec_slices(g.HP);
  r.waves = 8;
  r.max_wg_tiles = 1;
  if (r.rec_x0) r.g_in0 = 4;  // x as one zero-padded MFMA K chunk
  return r;
}

static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

PackedLayout packed_layout(const Geometry& g) {
  PackedLayout p;
  size_t off = 0;
  p.wpack = off;
  // HP / 16 gate-row groups x kc chunks of 64 lanes x 8 halfs per gate: the same size whether one
  // workgroup or `slices` workgroups hold a layer (the all-layers kernels only).
  if (g.wave_ok) off = align256(off + (size_t)g.L * (g.HP / 16) * g.kc * 4 * 64 * 8 * sizeof(_Float16));
  p.bias = off;
  off = align256(off + (size_t)g.L * 4 * g.HP * sizeof(float));
  p.wlin = off;
  off = align256(off + (size_t)g.O * g.HP * sizeof(float));
  p.blin = off;
  off = align256(off + (size_t)g.O * sizeof(float));
  // The layer-sequential kernel's W_hh alone (half of the above) and the projection GEMM's W_ih.
  p.wrec = off;
  if (g.rec_ok) off = align256(off + (size_t)g.L * (g.HP / 16) * g.kci * 4 * 64 * 8 * sizeof(_Float16));
  p.wih = off;
  if (g.rec_ok) off = align256(off + (size_t)4 * g.HP * (g.kp0 + (size_t)(g.L - 1) * g.kp) * sizeof(_Float16));
  p.wx0 = off;
  if (g.rec_ok && g.rec_x0) off = align256(off + (size_t)g.HP * 128 * sizeof(_Float16));
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
  w.xp = align256(w.counters + sizeof(uint32_t) * (size_t)g.L * ntile * counter_stride(g));
  if (g.rec) {
    // xp (rec_x0 only) holds x as [ntile][T][4][16] f16x8
    w.hseq = w.xring = align256(w.xp + (g.rec_x0 ? ntile * seq_len * 4 * 16 * 16 : 0));
    w.xring_words = ntile * (2 * g.HP * 8 + 16);  // the ring, then a 32-entry u32 XCD table per tile
    w.gates = align256(w.xring + w.xring_words * sizeof(uint64_t));
    w.xs = align256(w.gates + (size_t)seq_len * chunk_rows * 4 * g.HP * sizeof(_Float16));
    w.xin = align256(w.xs + (size_t)2 * seq_len * chunk_rows * g.HP * sizeof(_Float16));
    w.total = align256(w.xin + (g.kp0 > g.HP ? (size_t)seq_len * chunk_rows * g.kp0 * sizeof(_Float16) : 0));
    return w;
  }
  w.hseq = align256(w.xp + ntile * seq_len * g.g_in0 * tile_rows * 16);
  w.xring = align256(w.hseq + (size_t)(g.L - 1) * ntile * seq_len * g.kci * frag_bytes);
  // the rings, then a u32 table of the slices' XCD ids, up to 16 per (layer, tile)
  w.xring_words = g.slices > 1 ? (size_t)g.L * ntile * (2 * g.HP * 8 + 8) : 0;
  w.total = align256(w.xring + w.xring_words * sizeof(uint64_t));
  w.gates = w.xs = w.xin = w.total;
  return w;
}

static const void* recurrent_kernel(const Geometry& g, int tile_rows, bool ragged, int wg_tiles = 1,
                                    bool x0 = false) {
  if (g.rec) return tile_rows == 16 && wg_tiles == 1 ? rec_kernel(g.HP, x0) : nullptr;
  if (g.slices > 1) return tile_rows == 16 ? sliced_kernel(g.HP, wg_tiles) : nullptr;
  return wavefront_kernel(g.HP, tile_rows, ragged);
}

int recurrent_capacity(const Geometry& g, int tile_rows, hipError_t* err) {
  // The smallest occupancy of the variants (with and without lengths, every tile count, with and
  // without the in-kernel layer-0 projection where it exists), so any fits.
  int cap = 0;
  for (int v = 0; v < 2 * g.max_wg_tiles * (g.rec && g.rec_x0 ? 2 : 1); ++v) {
    const bool ragged = v & 1;
    const bool x0 = g.rec && (v / (2 * g.max_wg_tiles)) == 1;
    const void* fn = recurrent_kernel(g, tile_rows, ragged, 1 + (v / 2) % g.max_wg_tiles, x0);
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
  const void* fn = recurrent_kernel(g, a.tile_rows, a.lengths != nullptr, a.wg_tiles, a.wx0 != nullptr);
  if (!fn || a.wg_tiles < 1 || a.ntile % a.wg_tiles) return hipErrorInvalidValue;
  ForwardArgs args = a;
  void* params[] = {&args};
  // One layer per launch (layer-sequential) or every layer of the chunk at once.
  const unsigned grid = g.rec            ? std::max(a.ntile, a.ntile_grid) * g.slices
                        : g.slices > 1     ? std::max(a.L * a.ntile / a.wg_tiles, a.groups_grid) * g.slices
                                           : a.L * a.ntile;
  // An ordinary launch on the stream's own queue.  Co-residency of the grid comes from the caller:
  // plh_forward sizes every launch to at most the occupancy-derived capacity (recurrent_capacity),
  // and the launch starts after the stream's previous kernels have finished, so every workgroup is
  // dispatched at once; the kernels' waits are bounded, so a workgroup that were not resident would
  // end the launch with PLH_STATUS_TIMEOUT and NaN outputs, not a hang.  The kernels use no
  // grid-wide barrier.  (A cooperative launch, used before, ran each persistent kernel on a second
  // HSA queue of the runtime: ~11 us per hop between the two queues in kernel traces, twice per
  // forward, and that extra queue was the one runtime object of forward runs that GEMM-only runs
  // never created.)
  return hipLaunchKernel(fn, dim3(grid), dim3(g.waves * 64), params, 0, s);
}

}  // namespace plh
