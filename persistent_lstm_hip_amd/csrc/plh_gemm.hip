// plh_gemm.hip -- the time-parallel input projection of the layer-sequential path on CDNA4 (gfx950):
//
//     C[m][n] = sum_k X[m][k] * W[n][k]        fp16 operands, fp32 accumulation, fp16 result
//
// X is a layer's input sequence for every (step, row) of a launch ([T * rows][ldx], K-contiguous),
// W is that layer's W_ih ([N = 4 HP][K], K-contiguous, rows in the recurrent kernel's lane order),
// C the gate pre-activations the recurrent kernel reads a step ahead.  It restates the
// reference's per-layer torch::matmul of fp16 tensors (persistent_lstm_hip.cu:2988-2994, fp16
// result), written as a hand-written MFMA kernel instead of a library GEMM.
//
// Design (a 128-column slice of W over 512 K is 128 KB of LDS):
//   * weight-stationary: each workgroup owns one 128-column slice of W, loaded once into LDS in MFMA
//     fragment order when K <= 512 (for K > 512 the slice is held in K blocks of 512, reloaded in
//     turn for every m-tile between two barriers), and walks the 512-row m-tiles of its m-group; its
//     8 waves (two per SIMD) each
//     compute a 64 (m) x 128 (n) sub-tile with v_mfma_f32_16x16x32_f16 (4 x 8 accumulator tiles,
//     128 fp32 per lane), W as the MFMA's A operand and X as its B operand;
//   * X goes from global memory straight into the B-fragment registers (a lane's 8 consecutive k
//     of one row are one 16-byte load), through a ring of 4 k-steps of 32: the loads of step s + 3
//     are issued before the MFMAs of step s, across tile boundaries, so a load has three steps
//     (~3000 cycles with the other wave of the SIMD) to arrive; the waves never synchronise after
//     the weight load;
//   * W's rows are placed in the fragment blocks of an n-tile pair (2p, 2p + 1) so that lane l of
//     tile 2p + h holds n = 32 p + 8 (l / 16) + 4 h + 0..3: the lane's two accumulators are 8
//     consecutive n, stored as one 16-byte write (row m = l % 16);
//   * XCD-aware placement: workgroups are dispatched round-robin over the 8 XCDs (workgroup b on
//     XCD b % 8), and the n-slices of one m-group share an XCD, so each m-tile of X is read from
//     HBM about once into that XCD's L2 and then from L2 by the other slices;
//   * the result goes out with nontemporal stores (it is read back by another kernel, long after);
//   * two layouts of X and C: row-major ([M][ldx], [M][ldc]), or fragment-blocked: X as
//     [M / 16][ldx / 32][64 lanes][8] (block (mb, kc) holds rows 16 mb + l % 16, k = 32 kc + 8 (l / 16)
//     + 0..7 in lane l) and C as [M / 16][ldc / 32][64][8] (n = 32 g + 8 (l / 16) + 0..7).  A lane's
//     16 bytes then sit at lane * 16 of a 1 KB block, so every load and store instruction of a wave
//     moves 1 KB of whole cache lines (row-major: 16 rows x 64 B).  The layer-sequential path keeps
//     its layer inputs and projections blocked (the recurrent kernel writes and reads them so).
// Requirements (checked by the host): K % 128 == 0, K <= kGemmMaxKTotal, N % 128 == 0, ldx and ldc
// multiples of 8 (blocked: of 32, and M % 16 == 0), 16-byte aligned pointers.  Rows m >= M are not
// stored (their loads are clamped to row M - 1).
#include <algorithm>

#include "plh_device.h"

namespace plh {
namespace {

#ifndef PLH_GEMM_WAVES
#define PLH_GEMM_WAVES 8
#endif
#ifndef PLH_GEMM_RING
#define PLH_GEMM_RING 4
#endif
constexpr int kGemmWaves = PLH_GEMM_WAVES;            // waves per workgroup
constexpr int kGemmWM = 32 / kGemmWaves;              // 16-row m-tiles per wave
constexpr int kGemmBM = kGemmWaves * kGemmWM * 16;    // rows per m-tile of a workgroup (512)
constexpr int kGemmBN = 128;                          // columns per workgroup (its W slice)
constexpr int kGemmMaxK = 512;                        // W slice of 128 x 512 fp16 = 128 KB of LDS
constexpr int kGemmKbSteps = kGemmMaxK / 32;          // k-steps of one K block
constexpr int kRing = PLH_GEMM_RING;                  // X fragment ring depth (k-steps of 32)
constexpr int kGemmKStep = 32 * kRing;                // K granule
constexpr int kGemmThreads = kGemmWaves * 64;

// Row (within the 128-column slice) of W held by row i of the A fragment of n-tile nt.
__device__ __forceinline__ int gemm_w_row(int nt, int i) {
  return 32 * (nt >> 1) + 8 * (i >> 2) + 4 * (nt & 1) + (i & 3);
}

// KB: K > 512, the W slice held in K blocks of 512 (kGemmKbSteps k-steps) reloaded per m-tile.
template <bool BLK, bool KB>
__global__ void __launch_bounds__(kGemmThreads)
proj_gemm_kernel(const _Float16* __restrict__ X, long long ldx, const _Float16* __restrict__ W, int K,
                 _Float16* __restrict__ C, long long ldc, int M, int tiles_m, int n_slices, int m_groups) {
  constexpr int WM = kGemmWM;
  // W slice (or K block of it): [k-chunk of 32][n-tile 0..7][64 lanes] f16x8, k-chunk major.
  __shared__ f16x8 wl[kGemmMaxK / 32 * 8 * 64];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // Workgroup -> (n-slice, m-group): the n-slices of an m-group share the XCD b % 8.
  const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3;
  const int ns = idx % n_slices;
  const int mg = (idx / n_slices) * 8 + xcd;
  if (mg >= m_groups) return;
  const int n0 = ns * kGemmBN;
  const int KS = K / 32;  // k-steps per tile (a multiple of kRing)

  // K block kb of the W slice (k-steps 16 kb .. 16 kb + 15, fewer in a last partial block) into LDS.
  auto load_w = [&](int kb) {
    const int ks0 = kb * kGemmKbSteps;
    const int nks = KS - ks0 < kGemmKbSteps ? KS - ks0 : kGemmKbSteps;
    for (int e = threadIdx.x; e < nks * 8 * 64; e += kGemmThreads) {
      const int l = e & 63, nt = (e >> 6) & 7, kc = e >> 9;
      const int n = n0 + gemm_w_row(nt, l & 15);
      wl[e] = *reinterpret_cast<const f16x8*>(W + (size_t)n * K + (ks0 + kc) * 32 + (l >> 4) * 8);
    }
  };
  if constexpr (!KB) {
    load_w(0);  // the whole slice, once
    __syncthreads();
  }

  // m-tiles of this m-group: mg, mg + m_groups, ...
  int mt = mg;
  if (mt >= tiles_m) return;
  // X fragment a of k-step s of a tile: lane l reads row tile * BM + wave * 16 WM + 16 a + l % 16
  // (clamped to M - 1), k = 32 s + 8 (l / 16) .. + 7.
  const int lrow = wave * (16 * WM) + (lane & 15), lk = (lane >> 4) * 8;
  // Blocked: the fragment (16-row block mb, k-chunk kc) is 64 f16x8 at (mb * ldx / 32 + kc) * 64; the
  // returned pointer is that of kc = 0, and k-chunk kc is 64 f16x8 further per chunk.
  auto xptr = [&](int tile, int a) -> const f16x8* {
    if constexpr (BLK) {
      int mb = (tile * kGemmBM + wave * (16 * WM)) / 16 + a;
      mb = mb < M / 16 ? mb : M / 16 - 1;
      return reinterpret_cast<const f16x8*>(X) + (size_t)mb * (ldx / 32) * 64 + lane;
    }
    int m = tile * kGemmBM + lrow + 16 * a;
    m = m < M ? m : M - 1;
    return reinterpret_cast<const f16x8*>(X + (size_t)m * ldx + lk);
  };
  constexpr int kStepVec = BLK ? 64 : 4;  // f16x8 from one k-chunk of 32 to the next
  f16x8 xr[kRing][WM];
  // Flat step f = (tile index within this workgroup) * KS + k-step; loads of step f go to ring slot
  // f % kRing.  Prologue: steps 0 .. kRing - 2 of the first tile.
#pragma unroll
  for (int j = 0; j < kRing - 1; ++j)
#pragma unroll
    for (int a = 0; a < WM; ++a) xr[j][a] = xptr(mt, a)[j * kStepVec];

  for (;;) {
    const int nmt = mt + m_groups;
    const int pmt = nmt < tiles_m ? nmt : mt;  // prefetch target past the last tile: reload this one
    f32x4 acc[WM][8];
#pragma unroll
    for (int a = 0; a < WM; ++a)
#pragma unroll
      for (int b = 0; b < 8; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kq = 0; kq < KS; kq += kRing) {
      if constexpr (KB) {
        // A new K block of W: every wave is done with the previous one (its MFMAs read it from
        // registers loaded before them), then the block is loaded and visible to all.
        if (kq % kGemmKbSteps == 0) {
          __syncthreads();
          load_w(kq / kGemmKbSteps);
          __syncthreads();
        }
      }
#pragma unroll
      for (int j = 0; j < kRing; ++j) {
        // Prefetch flat step + kRing - 1 into its slot: this tile's k-step kq + j + kRing - 1, or the
        // next tile's first steps.
        {
          const int kn = kq + j + kRing - 1;
          const bool nxt = kn >= KS;
          const int t = nxt ? pmt : mt, kk = nxt ? kn - KS : kn;
#pragma unroll
          for (int a = 0; a < WM; ++a) xr[(j + kRing - 1) % kRing][a] = xptr(t, a)[kk * kStepVec];
        }
        const f16x8* wp = wl + (KB ? (kq + j) % kGemmKbSteps : kq + j) * 8 * 64 + lane;
        f16x8 wa[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) wa[b] = wp[b * 64];
#pragma unroll
        for (int a = 0; a < WM; ++a)
#pragma unroll
          for (int b = 0; b < 8; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[b], xr[j][a], acc[a][b], 0, 0, 0);
      }
    }
    // Lane holds rows mt * BM + lrow + 16 a and, for n-tile pair p, columns n0 + 32 p + 8 (lane / 16)
    // + 0..7.
    const int mrow = mt * kGemmBM + lrow;
    const int ncol = n0 + lk;
#pragma unroll
    for (int a = 0; a < WM; ++a) {
      const int m = mrow + 16 * a;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        f16x8 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] = (_Float16)acc[a][2 * p][j];
          v[4 + j] = (_Float16)acc[a][2 * p + 1][j];
        }
        // Nontemporal stores: the result streams to HBM without displacing the L2-resident X tiles the
        // other n-slices of the m-group still read (and is consumed by another kernel much later):
        // [512000,128]x[128,512] 0.148 -> 0.111 ms (4.4 -> 5.9 TB/s), [512000,512]x[512,2048]
        // 1.06 -> 1.03 ms, interleaved runs on one box.
        if (m < M) {
          if constexpr (BLK)
            __builtin_nontemporal_store(
                v, reinterpret_cast<f16x8*>(C) + ((size_t)(m >> 4) * (ldc / 32) + (n0 >> 5) + p) * 64 + lane);
          else
            __builtin_nontemporal_store(v, reinterpret_cast<f16x8*>(C + (size_t)m * ldc + ncol + 32 * p));
        }
      }
    }
    if (nmt >= tiles_m) break;
    mt = nmt;
  }
}

// The blocked layouts at K = 32 KS (KS = 4, 8, 12 or 16: K = 128, 256, 384, 512), with the k-steps of an m-tile
// unrolled at compile time.  The same work split, W slice and X ring as proj_gemm_kernel, written so
// that the compiler keeps the ring's loads kRing - 1 steps ahead everywhere: with a runtime k-loop the
// register allocator rotated the ring slots through the accumulators and waited for every
// outstanding load (vmcnt(0) / vmcnt(1)) twice per four k-steps.  Here
//   * X and C go through buffer descriptors of the wave's 64 rows, so a load or store is one
//     instruction with a scalar offset (16-row block a, k-chunk kc) and the lane's 16-byte offset:
//     no per-load 64-bit address arithmetic; blocks at or past M / 16 fall outside the descriptor,
//     so their loads read zeros and their stores are dropped (no clamping);
//   * the W fragments of a k-step are read from LDS two ahead of the MFMAs that use them (3 live
//     instead of 8), and scheduling groups fix each step's issue order: the ring's 4 loads, 2 W
//     reads, then 6 x (4 MFMAs, 1 W read) and 8 MFMAs;
//   * a tile's result is converted and stored during the next tile's first k-step, each pair of
//     column blocks right before that step's MFMAs overwrite its accumulators, instead of in an
//     epilogue during which the wave issues no MFMAs (the first tile stores through a descriptor
//     of no bytes, the last after the loop).
// [512000,512]x[512,2048] 1.03-1.05 -> 0.966-0.98 ms, [512000,128]x[128,512] 0.117 -> 0.109 ms
// (interleaved runs on one box each); the stores in the next tile's first step: 0.943-0.951 ->
// 0.933-0.935 ms and 0.105-0.106 -> 0.104-0.106 ms, bit-identical.
template <int KS>
__global__ void __launch_bounds__(kGemmThreads)
proj_gemm_blocked_kernel(const _Float16* __restrict__ X, long long ldx, const _Float16* __restrict__ W,
                         _Float16* __restrict__ C, long long ldc, int M, int tiles_m, int n_slices, int m_groups) {
  static_assert(kGemmWaves == 8 && kGemmWM == 4 && KS % kRing == 0 && KS * 32 <= kGemmMaxK, "tile shape");
  constexpr int K = 32 * KS;
  __shared__ f16x8 wl[KS * 8 * 64];  // [k-chunk][n-tile 0..7][64 lanes] f16x8
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int xcd = blockIdx.x & 7, idx = blockIdx.x >> 3;
  const int ns = idx % n_slices;
  const int mg = (idx / n_slices) * 8 + xcd;
  if (mg >= m_groups) return;
  const int n0 = ns * kGemmBN;
  for (int e = threadIdx.x; e < KS * 8 * 64; e += kGemmThreads) {
    const int l = e & 63, nt = (e >> 6) & 7, kc = e >> 9;
    const int n = n0 + gemm_w_row(nt, l & 15);
    wl[e] = *reinterpret_cast<const f16x8*>(W + (size_t)n * K + kc * 32 + (l >> 4) * 8);
  }
  __syncthreads();
  int mt = mg;
  if (mt >= tiles_m) return;
  const int nblk = M / 16;
  const int xa = (int)(ldx * 32), ca = (int)(ldc * 32);  // bytes from one 16-row block to the next
  // 16-row blocks a descriptor may span (its byte count is a 31-bit number)
  const int max_xb = 0x7FFFFFFF / xa, max_cb = 0x7FFFFFFF / ca;
  // X rows of m-tile t held by this wave: blocks 32 t + 4 wave .. + 3
  auto xrs = [&](int t) {
    const int mb = t * (kGemmBM / 16) + wave * kGemmWM;
    const int nb = min(max(nblk - mb, 0), max_xb);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(X) + (size_t)(mb < nblk ? mb : 0) * ldx * 16, 0,
                                             nb * xa, 0x00020000);
  };
  const unsigned voff = (unsigned)lane * 16u;
  f16x8 xr[kRing][kGemmWM];
  auto ld = [&](__amdgpu_buffer_rsrc_t rs, int kc, f16x8 (&dst)[kGemmWM]) {
#pragma unroll
    for (int a = 0; a < kGemmWM; ++a)
      dst[a] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, a * xa + kc * 1024, 0));
  };
  {
    // In ring order, as the loop's last steps issue them for the next tile: the loop header's waits
    // are the tighter of the two paths into it, and a slot loaded last here would make every tile's
    // first step wait for the previous tile's result stores.
    const auto rs = xrs(mt);
#pragma unroll
    for (int j = 0; j < kRing - 1; ++j) {
      ld(rs, j, xr[j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  f32x4 acc[kGemmWM][8];
  // k-step s of the tile whose X rows rc describes (rn: the next tile's, for the ring's loads past
  // this tile's last step).  Step 0 starts every accumulator from zero; with `out` (a fused step 0)
  // each accumulator pair of the previous tile is converted and stored right before the step's
  // MFMAs overwrite it, so the epilogue's VALU work and stores run beside the next tile's first
  // MFMAs instead of stalling the matrix core.
  auto kstep = [&](int s, __amdgpu_buffer_rsrc_t rc, __amdgpu_buffer_rsrc_t rn, const __amdgpu_buffer_rsrc_t* out)
      __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    {
      const int sn = s + kRing - 1;  // this tile's step sn, or the next tile's first steps
      if (sn < KS)
        ld(rc, sn, xr[sn % kRing]);
      else
        ld(rn, sn - KS, xr[sn % kRing]);
    }
    f16x8 wa[3];
    wa[0] = wl[(s * 8 + 0) * 64 + lane];
    wa[1] = wl[(s * 8 + 1) * 64 + lane];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      if (b + 2 < 8) wa[(b + 2) % 3] = wl[(s * 8 + b + 2) * 64 + lane];
      if (out && b % 2 == 0) {
        // the previous tile's column blocks n0 / 32 + b / 2: blocks 32 mt + 4 wave + a
#pragma unroll
        for (int a = 0; a < kGemmWM; ++a) {
          f16x8 v;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            v[j] = (_Float16)acc[a][b][j];
            v[4 + j] = (_Float16)acc[a][b + 1][j];
          }
          // nontemporal (cache policy 2), as in proj_gemm_kernel
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v),
                                                 *out, voff, a * ca + (b / 2) * 1024, 2);
        }
      }
#pragma unroll
      for (int a = 0; a < kGemmWM; ++a)
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[b % 3], xr[s % kRing][a],
                                                          s == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[a][b], 0, 0, 0);
    }
    // issue order (masks: 0x020 vector-memory reads, 0x100 LDS reads, 0x008 MFMA, 0x002 VALU,
    // 0x040 vector-memory writes)
    __builtin_amdgcn_sched_group_barrier(0x020, kGemmWM, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    if (!out) {
#pragma unroll
      for (int g = 0; g < 6; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, kGemmWM, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * kGemmWM, 0);
    } else {
      // per pair of column blocks: the conversions and stores of the previous tile's pair, then
      // the MFMAs that overwrite it (each with the W read two blocks ahead)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x002, 4 * kGemmWM, 0);
        __builtin_amdgcn_sched_group_barrier(0x040, kGemmWM, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, kGemmWM, 0);
        if (g < 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, kGemmWM, 0);
        if (g < 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
  };
  // the result descriptor of tile t: blocks 32 t + 4 wave + a, column blocks n0 / 32 + p; rows at or
  // past M fall outside it
  auto crs = [&](int t) {
    const int mb = t * (kGemmBM / 16) + wave * kGemmWM;
    const int rem = max(min(max(nblk - mb, 0), max_cb) * ca - n0 * 32, 0);
    return __builtin_amdgcn_make_buffer_rsrc(C + (mb < nblk ? (size_t)mb * ldc * 16 + (size_t)n0 * 16 : 0), 0, rem,
                                             0x00020000);
  };
  // The previous tile's result descriptor: none before the first tile (its stores are dropped).
  __amdgpu_buffer_rsrc_t prev = __builtin_amdgcn_make_buffer_rsrc(C, 0, 0, 0x00020000);
#pragma unroll
  for (int a = 0; a < kGemmWM; ++a)
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (;;) {
    const int nmt = mt + m_groups;
    const int pmt = nmt < tiles_m ? nmt : mt;  // prefetch target past the last tile: reload this one
    const auto rc = xrs(mt), rn = xrs(pmt);
    kstep(0, rc, rn, &prev);
#pragma unroll
    for (int s = 1; s < KS; ++s) kstep(s, rc, rn, nullptr);
    __builtin_amdgcn_sched_barrier(0);
    prev = crs(mt);
    if (nmt >= tiles_m) break;
    mt = nmt;
  }
#pragma unroll
  for (int a = 0; a < kGemmWM; ++a)
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      f16x8 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = (_Float16)acc[a][2 * p][j];
        v[4 + j] = (_Float16)acc[a][2 * p + 1][j];
      }
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v),
                                             prev, voff, a * ca + p * 1024, 2);
    }
}

}  // namespace

bool gemm_shape_ok(long long M, int N, int K, long long ldx, long long ldc, bool blocked) {
  const int q = blocked ? 32 : 8;
  return M >= 0 && N > 0 && K > 0 && N % kGemmBN == 0 && K % kGemmKStep == 0 && K <= kGemmMaxKTotal && ldx >= K &&
         ldc >= N && ldx % q == 0 && ldc % q == 0 && (!blocked || M % 16 == 0) && M <= (long long)INT32_MAX;
}

hipError_t launch_proj_gemm(const _Float16* X, long long ldx, const _Float16* W, int K, _Float16* C, long long ldc,
                            long long M, int N, bool blocked, int cus, hipStream_t s) {
  if (!gemm_shape_ok(M, N, K, ldx, ldc, blocked)) return hipErrorInvalidValue;
  if (M == 0) return hipSuccess;
  const int tiles_m = (int)((M + kGemmBM - 1) / kGemmBM), n_slices = N / kGemmBN;
  // One workgroup per CU: n_slices per m-group, as many m-groups as fill the device (at most one per
  // m-tile), placed so that an m-group's slices share an XCD.
  const int m_groups = std::max(1, std::min(tiles_m, std::max(cus, 1) / n_slices));
  const int grid = ((m_groups + 7) / 8) * 8 * n_slices;
  // The compile-time-K kernel where one is built (other K: the generic kernel).
  auto* fk = !blocked || ldc > (1 << 20) ? nullptr
             : K == 128                   ? proj_gemm_blocked_kernel<4>
             : K == 256                   ? proj_gemm_blocked_kernel<8>
             : K == 384                   ? proj_gemm_blocked_kernel<12>
             : K == 512                   ? proj_gemm_blocked_kernel<16>
                                          : nullptr;
  if (fk) {
    hipLaunchKernelGGL(fk, dim3(grid), dim3(kGemmThreads), 0, s, X, ldx, W, C, ldc, (int)M, tiles_m, n_slices, m_groups);
    return hipGetLastError();
  }
  const bool kb = K > kGemmMaxK;
  auto* fn = blocked ? (kb ? proj_gemm_kernel<true, true> : proj_gemm_kernel<true, false>)
                     : (kb ? proj_gemm_kernel<false, true> : proj_gemm_kernel<false, false>);
  hipLaunchKernelGGL(fn, dim3(grid), dim3(kGemmThreads), 0, s, X, ldx, W, K, C, ldc, (int)M, tiles_m, n_slices,
                     m_groups);
  return hipGetLastError();
}

double proj_gemm_flops(long long M, int N, int K) { return 2.0 * (double)M * N * K; }

}  // namespace plh
