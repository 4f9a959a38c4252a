// plh_capi.hip -- extern "C" entry points declared in include/persistent_lstm_hip.h.
//
// Argument checking follows the reference's boundary (persistent_lstm_op.cpp:7-11 raises
// std::invalid_argument for bad shapes; persistent_lstm_hip.cu:1730-1735 turns HIP errors into
// std::runtime_error): here they become PLH_ERR_INVALID / PLH_ERR_HIP plus a message.  Unlike the
// reference there is no silent fallback: a geometry the kernels do not implement is an error.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "plh_internal.h"
#include "../../include/persistent_lstm_hip.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int fail_hip(hipError_t e, const char* what) {
  return fail(PLH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Co-resident workgroup capacity per (device, HP, tile rows, path), queried once.
std::mutex g_cap_mu;
std::unordered_map<long long, int> g_cap;

int capacity(const plh::Geometry& g, int tile_rows, hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return 0;
  const long long key = (((long long)dev * 4096 + g.HP) * 64 + tile_rows) * 2 + g.rec;
  {
    std::lock_guard<std::mutex> lk(g_cap_mu);
    auto it = g_cap.find(key);
    if (it != g_cap.end()) return it->second;
  }
  const int c = plh::recurrent_capacity(g, tile_rows, err);
  if (*err != hipSuccess) return 0;
  std::lock_guard<std::mutex> lk(g_cap_mu);
  g_cap[key] = c;
  return c;
}

// Launch plan: every (layer, tile, slice) workgroup of one persistent launch must be co-resident.
// 8-row tiles halve the gate math per workgroup and are used when the whole batch fits one launch
// with them; otherwise 16-row tiles, and the batch is split into sequential launches if needed.
// Sliced geometries (HP 256, 512) always use 16-row tiles; the layer-sequential one (HP 512) needs only
// the workgroups of one layer co-resident.
struct Plan {
  int tile_rows = 16;
  int chunk_rows = 16;
  int wg_tiles = 1;  // sliced: 16-row tiles per workgroup
  bool rec = false;  // layer-sequential path (plh::as_layer_sequential)
  bool fits = true;  // the workgroups of one tile fit the device at once
  bool pad8 = false; // the co-resident tiles are a multiple of 8: a launch may round its grid up to 8 tiles
  int cap_wgs = 0;   // co-resident workgroups (16-row tiles)
};

Plan make_plan(const plh::Geometry& g, int batch, int cap8, int cap16) {
  Plan p;
  batch = std::max(batch, 1);
  const int tiles8 = (batch + 7) / 8;
  if (g.slices == 1 && (long long)g.L * tiles8 <= cap8) {
    p.tile_rows = 8;
    p.chunk_rows = tiles8 * 8;
    return p;
  }
  // Workgroups per layer of one launch; where the launch is large enough, a multiple of 8 of them
  // keeps the XCD-aware mapping available.  A sliced workgroup carries two software-pipelined tiles
  // (where the kernel allows it) only when one tile each would need more than one launch.
  int groups = cap16 / (g.rec ? g.slices : g.L * g.slices);
  p.fits = groups >= 1;
  if (groups >= 8) groups &= ~7;
  p.pad8 = groups >= 8;  // (then a multiple of 8)
  p.cap_wgs = cap16;
  groups = std::max(1, groups);
  const int tiles16 = (batch + 15) / 16;
  const int wt = (g.slices > 1 && g.max_wg_tiles > 1 && tiles16 > groups) ? g.max_wg_tiles : 1;
  const int tiles = std::min(groups * wt, (tiles16 + wt - 1) / wt * wt);
  p.tile_rows = 16;
  p.chunk_rows = tiles * 16;
  p.wg_tiles = wt;
  return p;
}

// Plan on the current device; without one (capacity unknown) assume one workgroup per CU of a
// 256-CU MI355X.
Plan plan_path(const plh::Geometry& g, int batch, bool need_device, hipError_t* err) {
  int cap8 = g.slices == 1 ? capacity(g, 8, err) : 0;
  int cap16 = *err == hipSuccess ? capacity(g, 16, err) : 0;
  if (*err != hipSuccess) {
    if (need_device) return Plan();
    cap8 = cap16 = 256;
    *err = hipSuccess;
  }
  return make_plan(g, batch, cap8, cap16);
}

// Where both paths exist (HP = 512), a fixed rule on step counts picks one: the wavefront path runs
// T + L - 1 steps per launch of all L layers, the layer-sequential path L x T steps per launch of up
// to 512 rows of one layer (plus one projection GEMM per layer after the first).  The
// layer-sequential path is used when the batch needs more wavefront launches than there are layers
// (so it does fewer launches of recurrent steps), and only while its workspace - a layer's
// projections for every step, ~4 MB per step at 512 rows - stays within kMaxSeqWorkspace.  It is also
// used whenever one tile of all L layers does not fit the device (L x 16 slices > the co-resident
// workgroups: more than 16 layers at padded H 512).
constexpr size_t kMaxSeqWorkspace = (size_t)24 << 30;
Plan plan_for(const plh::Geometry& g, int batch, int seq_len, bool need_device, hipError_t* err) {
  if (!g.wave_ok) {
    // Padded H 1024, or an input wider than the padded H: only the layer-sequential path exists.
    Plan q = plan_path(plh::as_layer_sequential(g), batch, need_device, err);
    q.rec = true;
    return q;
  }
  const Plan p = plan_path(g, batch, need_device, err);
  if (!g.rec_ok || *err != hipSuccess) return p;
  const plh::Geometry gr = plh::as_layer_sequential(g);
  Plan q = plan_path(gr, batch, need_device, err);
  if (*err != hipSuccess) return p;
  q.rec = true;
  if (plh::workspace_layout(gr, seq_len, q.chunk_rows, q.tile_rows).total > kMaxSeqWorkspace) return p;
  if (!p.fits) return q;
  const long long n_wave = (std::max(batch, 1) + (long long)p.chunk_rows - 1) / p.chunk_rows;
  return n_wave > g.L ? q : p;
}

bool geometry(int I, int H, int L, int O, plh::Geometry* g) {
  std::string why;
  if (!plh::make_geometry(I, H, L, O, g, &why)) {
    g_last_error = why;
    return false;
  }
  return true;
}

int geometry_code(int I, int H, int L, int O) {
  return (I <= 0 || H <= 0 || L <= 0 || O < 0) ? PLH_ERR_INVALID : PLH_ERR_UNSUPPORTED;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Armed timing events of the calling thread (plh_kernel_timing).  Held through a pointer that is
// never deleted: a thread_local object's destructor would run at thread or process exit, possibly
// after the HIP runtime has been torn down, so the library makes no HIP call from a destructor.
// Events are released only by plh_kernel_timing() itself (re-arming or disarming).
struct KernelTiming {
  std::vector<hipEvent_t> ev;  // begin/end pairs
  int used = 0;                // pairs recorded
  void release() {
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
    ev.clear();
    used = 0;
  }
};
thread_local KernelTiming* g_timing_ptr = nullptr;
KernelTiming& timing() {
  if (!g_timing_ptr) g_timing_ptr = new KernelTiming();
  return *g_timing_ptr;
}

// Bound on inter-workgroup waits of this thread's forwards (plh_set_wait_limit_us).
constexpr int64_t kDefaultWaitUs = 2000000;
thread_local int64_t g_wait_us = kDefaultWaitUs;
// Failure injection of this thread's forwards (plh_inject_wait_failure); -1: off.
thread_local int g_fail_step = -1;

// Compute units of the current device (the persistent projection GEMM's grid), queried once per
// device.
std::mutex g_cus_mu;
std::unordered_map<int, int> g_cus;

int device_cus(hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return 0;
  {
    std::lock_guard<std::mutex> lk(g_cus_mu);
    auto it = g_cus.find(dev);
    if (it != g_cus.end()) return it->second;
  }
  int cus = 0;
  *err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (*err != hipSuccess) return 0;
  std::lock_guard<std::mutex> lk(g_cus_mu);
  g_cus[dev] = cus;
  return cus;
}

// Device scratch of plh_forward_noalloc: one copy on every GPU the library runs on, held until the
// process ends.  In host code `scratch` names a host-side stand-in, not a device address: host code
// uses only the per-device address from hipGetSymbolAddress (scratch_ptr).
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::unordered_map<int, void*> g_scratch;

// The device address of `scratch` on the current device, looked up once per device.
void* scratch_ptr(hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch.find(dev);
  if (it != g_scratch.end()) return it->second;
  void* ptr = nullptr;
  *err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (*err != hipSuccess) return nullptr;
  g_scratch[dev] = ptr;
  return ptr;
}

// Forwards on different streams of one device run one after the other.  Each persistent launch needs
// all its workgroups co-resident; two launched from two streams at once would be dispatched
// interleaved, each holding part of the device while waiting for its own undispatched workgroups,
// until both time out.  While a device has seen forwards on one stream only, that stream orders
// them and nothing else is done (an event record per forward costs ~3.5 us of the next launch).
// The first forward on a second stream synchronises the device once (the earlier stream's handle
// may be gone, so no event is recorded on it); from then on each forward waits (hipStreamWaitEvent)
// for the device's last forward when that one was on another stream, and records an event after
// its own launches.  Inside a stream capture nothing is waited for or recorded: the captured
// graph's launches are ordered by whoever replays it.
struct DeviceOrder {
  std::mutex mu;
  hipEvent_t done = nullptr;   // multi: recorded after the last forward's launches (never destroyed)
  hipStream_t last = nullptr;  // the stream of the last forward (compared, never used)
  bool any = false;            // a forward was enqueued
  bool multi = false;          // forwards were enqueued on more than one stream
};
std::mutex g_order_mu;
std::unordered_map<int, DeviceOrder*> g_order;  // one per device, never freed

class StreamOrder {
 public:
  explicit StreamOrder(hipStream_t s) : s_(s) {
    int dev = 0;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    err_ = hipGetDevice(&dev);
    if (err_ == hipSuccess) err_ = hipStreamIsCapturing(s, &cs);
    if (err_ != hipSuccess || cs != hipStreamCaptureStatusNone) return;
    {
      std::lock_guard<std::mutex> lk(g_order_mu);
      DeviceOrder*& o = g_order[dev];
      if (!o) o = new DeviceOrder();
      order_ = o;
    }
    lock_ = std::unique_lock<std::mutex>(order_->mu);
    const bool other = order_->any && order_->last != s;
    if (other && !order_->multi) {
      if (!order_->done) err_ = hipEventCreateWithFlags(&order_->done, hipEventDisableTiming);
      if (err_ == hipSuccess) err_ = hipDeviceSynchronize();
      if (err_ != hipSuccess) return;
      order_->multi = true;
    } else if (other) {
      err_ = hipStreamWaitEvent(s, order_->done, 0);
      if (err_ != hipSuccess) return;
    }
    active_ = true;
  }
  hipError_t error() const { return err_; }
  // After the forward's launches (also after a failed one: what it enqueued is ordered too).
  ~StreamOrder() {
    if (!active_) return;
    if (order_->multi && hipEventRecord(order_->done, s_) != hipSuccess) return;
    order_->last = s_;
    order_->any = true;
  }

 private:
  hipStream_t s_;
  DeviceOrder* order_ = nullptr;
  std::unique_lock<std::mutex> lock_;
  hipError_t err_ = hipSuccess;
  bool active_ = false;
};

}  // namespace

extern "C" {

int plh_abi_version(void) { return 1; }

const char* plh_last_error(void) { return g_last_error.c_str(); }

int plh_supports(int input_size, int hidden_size, int num_layers, int output_size) {
  plh::Geometry g;
  return geometry(input_size, hidden_size, num_layers, output_size, &g) ? 1 : 0;
}

int64_t plh_packed_bytes(int input_size, int hidden_size, int num_layers, int output_size) {
  plh::Geometry g;
  if (!geometry(input_size, hidden_size, num_layers, output_size, &g)) return -1;
  return (int64_t)plh::packed_layout(g).total;
}

int plh_pack_regressor(int input_size, int hidden_size, int num_layers, int output_size,
                       const void* const* w_ih, const void* const* w_hh, const void* const* b_ih,
                       const void* const* b_hh, const void* lin_w, const void* lin_b, void* packed_dev,
                       int64_t packed_bytes, void* stream) {
  plh::Geometry g;
  if (!geometry(input_size, hidden_size, num_layers, output_size, &g))
    return geometry_code(input_size, hidden_size, num_layers, output_size);
  const plh::PackedLayout p = plh::packed_layout(g);
  if (!packed_dev || packed_bytes < (int64_t)p.total)
    return fail(PLH_ERR_INVALID, "packed buffer missing or smaller than plh_packed_bytes()");
  if (!aligned(packed_dev, 256)) return fail(PLH_ERR_INVALID, "packed buffer must be 256-byte aligned");
  if (!w_ih || !w_hh || !b_ih) return fail(PLH_ERR_INVALID, "w_ih, w_hh and b_ih arrays are required");
  if (output_size > 0 && !lin_w) return fail(PLH_ERR_INVALID, "lin_w is required when output_size > 0");
  hipStream_t s = (hipStream_t)stream;
  char* base = (char*)packed_dev;
  size_t wih_off = p.wih;
  for (int l = 0; l < g.L; ++l) {
    if (!w_ih[l] || !w_hh[l]) return fail(PLH_ERR_INVALID, "null weight pointer for layer " + std::to_string(l));
    hipError_t e = hipSuccess;
    if (g.wave_ok) {
      e = plh::launch_pack_layer(g, l, (const _Float16*)w_ih[l], (const _Float16*)w_hh[l],
                                 (_Float16*)(base + p.wpack), s);
      if (e != hipSuccess) return fail_hip(e, "pack_layer launch");
    }
    if (g.rec_ok) {
      // The layer-sequential path's operands: W_hh fragments; W_ih as the projection GEMM's W operand,
      // or for layer 0 with I <= 32 as the recurrent kernel's MFMA fragments.
      e = plh::launch_pack_rec_layer(g, l, (const _Float16*)w_hh[l], (_Float16*)(base + p.wrec), s);
      if (e != hipSuccess) return fail_hip(e, "pack_rec_layer launch");
      if (l == 0 && g.rec_x0) {
        e = plh::launch_pack_rec_wx0(g, (const _Float16*)w_ih[0], (_Float16*)(base + p.wx0), s);
        if (e != hipSuccess) return fail_hip(e, "pack_rec_wx0 launch");
      } else {
        const int K = l == 0 ? g.I : g.H, Kp = l == 0 ? g.kp0 : g.kp;
        e = plh::launch_pack_rec_wih(g, (const _Float16*)w_ih[l], K, Kp, (_Float16*)(base + wih_off), s);
        if (e != hipSuccess) return fail_hip(e, "pack_rec_wih launch");
        wih_off += (size_t)4 * g.HP * Kp * sizeof(_Float16);
      }
    }
    e = plh::launch_pack_bias(g, l, (const _Float16*)b_ih[l], b_hh ? (const _Float16*)b_hh[l] : nullptr,
                              (float*)(base + p.bias), s);
    if (e != hipSuccess) return fail_hip(e, "pack_bias launch");
  }
  hipError_t e = plh::launch_pack_linear(g, (const _Float16*)lin_w, (const _Float16*)lin_b,
                                         (float*)(base + p.wlin), (float*)(base + p.blin), s);
  if (e != hipSuccess) return fail_hip(e, "pack_linear launch");
  return PLH_OK;
}

int64_t plh_workspace_bytes(int input_size, int hidden_size, int num_layers, int output_size, int batch,
                            int seq_len) {
  plh::Geometry g;
  if (!geometry(input_size, hidden_size, num_layers, output_size, &g)) return -1;
  if (batch < 0 || seq_len < 0) {
    g_last_error = "batch and seq_len must be non-negative";
    return -1;
  }
  hipError_t err = hipSuccess;
  const Plan p = plan_for(g, batch, seq_len, false, &err);
  if (p.rec) g = plh::as_layer_sequential(g);
  return (int64_t)plh::workspace_layout(g, seq_len, p.chunk_rows, p.tile_rows).total;
}

int plh_forward(const void* packed_dev, int input_size, int hidden_size, int num_layers, int output_size,
                const void* x, int batch, int seq_len, const int32_t* lengths, const void* h0, const void* c0,
                void* out, void* out_seq, void* h_n, void* c_n, const int32_t* probe_steps, int n_probe,
                float* probe_h, float* probe_c, void* workspace, int64_t workspace_bytes, void* stream) {
  plh::Geometry g;
  if (!geometry(input_size, hidden_size, num_layers, output_size, &g))
    return geometry_code(input_size, hidden_size, num_layers, output_size);
  if (batch < 0 || seq_len < 0) return fail(PLH_ERR_INVALID, "batch and seq_len must be non-negative");
  if (!packed_dev) return fail(PLH_ERR_INVALID, "packed weights are required");
  if (batch > 0 && seq_len > 0 && !x) return fail(PLH_ERR_INVALID, "x is required");
  if (n_probe < 0 || (n_probe > 0 && (!probe_steps || !probe_h || !probe_c)))
    return fail(PLH_ERR_INVALID, "probe_steps, probe_h and probe_c are required when n_probe > 0");
  if (n_probe > seq_len) return fail(PLH_ERR_INVALID, "more probe steps than sequence steps");
  if (!workspace || !aligned(workspace, 256)) return fail(PLH_ERR_INVALID, "workspace must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;

  hipError_t err = hipSuccess;
  const Plan plan = plan_for(g, batch, seq_len, true, &err);
  if (err != hipSuccess) return fail_hip(err, "occupancy query");
  if (plan.rec) g = plh::as_layer_sequential(g);
  const int tile_wgs = g.rec ? g.slices : g.L * g.slices;
  if (capacity(g, 16, &err) < tile_wgs)
    return fail(PLH_ERR_UNSUPPORTED, "the device cannot hold the " + std::to_string(tile_wgs) +
                                         " workgroups of one batch tile co-resident (layers = " +
                                         std::to_string(g.L) + ")");
  const int chunk_rows = plan.chunk_rows;
  const plh::WorkspaceLayout w = plh::workspace_layout(g, seq_len, chunk_rows, plan.tile_rows);
  if (workspace_bytes < (int64_t)w.total)
    return fail(PLH_ERR_INVALID, "workspace smaller than plh_workspace_bytes()");

  const plh::PackedLayout p = plh::packed_layout(g);
  char* ws = (char*)workspace;
  const char* pk = (const char*)packed_dev;
  uint32_t* status = (uint32_t*)(ws + w.status);
  uint32_t* counters = (uint32_t*)(ws + w.counters);

  StreamOrder order(s);
  if (order.error() != hipSuccess) return fail_hip(order.error(), "ordering against other streams' forwards");
  if (batch == 0) {
    err = plh::launch_zero_u32(status, 1, s);
    return err == hipSuccess ? PLH_OK : fail_hip(err, "status reset");
  }

  plh::ForwardArgs a;
  std::memset(&a, 0, sizeof(a));
  a.x = (const _Float16*)x;
  a.lengths = lengths;
  a.wpack = (const _Float16*)(pk + (g.rec ? p.wrec : p.wpack));
  a.bias = (const float*)(pk + p.bias);
  a.wlin = (const float*)(pk + p.wlin);
  a.blin = (const float*)(pk + p.blin);
  a.xp = (plh::f16x8_t*)(ws + w.xp);
  a.hseq = (plh::f16x8_t*)(ws + w.hseq);
  a.xring = (uint64_t*)(ws + w.xring);
  a.counters = counters;
  a.status = status;
  a.h0 = (const _Float16*)h0;
  a.c0 = (const _Float16*)c0;
  a.out = output_size > 0 ? (_Float16*)out : nullptr;
  a.out_seq = (_Float16*)out_seq;
  a.h_n = (_Float16*)h_n;
  a.c_n = (_Float16*)c_n;
  a.probe_steps = probe_steps;
  a.probe_h = probe_h;
  a.probe_c = probe_c;
  a.n_probe = n_probe;
  a.B = batch;
  a.T = seq_len;
  a.I = g.I;
  a.H = g.H;
  a.L = g.L;
  a.O = g.O;
  a.g_in0 = g.g_in0;
  a.wait_ticks = (uint64_t)g_wait_us * 100u;  // s_memrealtime: 100 MHz
  a.fail_step = g_fail_step;

  KernelTiming& tm = timing();
  const bool timed = tm.used * 2 < (int)tm.ev.size();
  const int cus = g.rec ? device_cus(&err) : 0;
  if (err != hipSuccess) return fail_hip(err, "device query");
  for (int row0 = 0; row0 < batch; row0 += chunk_rows) {
    const int rows = std::min(chunk_rows, batch - row0);
    a.row0 = row0;
    a.row_end = row0 + rows;
    a.tile_rows = plan.tile_rows;
    a.ntile = (rows + plan.tile_rows - 1) / plan.tile_rows;
    a.wg_tiles = plan.wg_tiles;
    a.ntile = (a.ntile + a.wg_tiles - 1) / a.wg_tiles * a.wg_tiles;
    a.rows_pad = a.ntile * plan.tile_rows;
    // Layer by layer, the grid covers a multiple of 8 tiles where the device holds that many (the
    // extra workgroups exit at once), so that every tile's slices share an XCD and exchange h through
    // its L2 whatever the batch: without it, B = 320 and 448 (20 and 28 tiles) took 10.2 and 11.2 ms
    // at H 512 against 9.3 ms at B = 384 (24 tiles).
    // The all-layers sliced kernel likewise rounds its (layer, tile group) groups up to a multiple
    // of 8 where the device holds them (H256 B200: 1.92 ms against 1.47 at B192).
    a.ntile_grid = g.rec && plan.pad8 ? (a.ntile + 7) / 8 * 8 : a.ntile;
    const int groups = g.L * a.ntile / a.wg_tiles, groups8 = (groups + 7) / 8 * 8;
    a.groups_grid = g.slices > 1 && !g.rec && groups8 * g.slices <= plan.cap_wgs ? groups8 : groups;
    a.xcd_map = ((g.slices > 1 && !g.rec) ? a.groups_grid % 8 : a.ntile_grid % 8) == 0 ? 1 : 0;
    if (g.rec) {
      // Layer by layer.  Layer 0: with I <= 32 its input projection runs inside the recurrent kernel
      // from x packed by the prologue; otherwise x goes to xs slot 0 for the projection GEMM.  Every
      // later layer: the projection GEMM of every step (plh_gemm.hip) over the previous layer's h
      // sequence, then the recurrent kernel, whose h sequence goes to the other xs slot.  The
      // exchange ring is cleared before each layer's launch (tags restart at 1).
      _Float16* xs[2] = {(_Float16*)(ws + w.xs),
                         (_Float16*)(ws + w.xs) + (size_t)seq_len * chunk_rows * g.HP};
      _Float16* gates = (_Float16*)(ws + w.gates);
      err = plh::launch_forward_prologue(g, a, row0 == 0 ? status : nullptr, g.rec_x0 ? 4 : 0, w.xring_words, s);
      if (err != hipSuccess) return fail_hip(err, "forward prologue");
      if (timed && row0 == 0) {
        err = hipEventRecord(tm.ev[2 * tm.used], s);
        if (err != hipSuccess) return fail_hip(err, "timing event");
      }
      // x for layer 0's GEMM: in xs slot 0, or (input wider than the padded H) in its own buffer
      _Float16* const xin = g.kp0 > g.HP ? (_Float16*)(ws + w.xin) : xs[0];
      const int ld0 = g.kp0 > g.HP ? g.kp0 : g.HP;
      if (!g.rec_x0) {
        err = plh::launch_rec_input(g, a, xin, ld0, s);
        if (err != hipSuccess) return fail_hip(err, "input transpose");
      }
      const _Float16* wih = (const _Float16*)(pk + p.wih);
      a.gates = gates;
      for (int l = 0; l < g.L; ++l) {
        const bool x0 = l == 0 && g.rec_x0;
        if (!x0) {
          const int Kp = l == 0 ? g.kp0 : g.kp;
          err = plh::launch_proj_gemm(l == 0 ? xin : xs[l & 1], l == 0 ? ld0 : g.HP, wih, Kp, gates, 4 * g.HP,
                                      (long long)seq_len * a.rows_pad, 4 * g.HP, true, cus, s);
          if (err != hipSuccess) return fail_hip(err, "input projection GEMM launch");
          wih += (size_t)4 * g.HP * Kp;
        }
        if (l > 0) {
          err = plh::launch_zero_u32((uint32_t*)a.xring, w.xring_words * 2, s);
          if (err != hipSuccess) return fail_hip(err, "exchange ring reset");
        }
        a.layer = l;
        a.hout = l + 1 < g.L ? xs[(l + 1) & 1] : nullptr;
        a.wx0 = x0 ? (const _Float16*)(pk + p.wx0) : nullptr;
        err = plh::launch_recurrent(g, a, s);
        if (err != hipSuccess) return fail_hip(err, "persistent LSTM launch");
      }
      a.wx0 = nullptr;
      continue;
    }
    // x of this launch's rows into xp; status (first launch), counters and, when sliced, the
    // exchange ring (tags restart at 1) cleared: one launch ahead of the persistent one
    err = plh::launch_forward_prologue(g, a, row0 == 0 ? status : nullptr, g.g_in0, w.xring_words, s);
    if (err != hipSuccess) return fail_hip(err, "forward prologue");
    if (timed && row0 == 0) {
      err = hipEventRecord(tm.ev[2 * tm.used], s);
      if (err != hipSuccess) return fail_hip(err, "timing event");
    }
    err = plh::launch_recurrent(g, a, s);
    if (err != hipSuccess) return fail_hip(err, "persistent LSTM launch");
  }
  if (timed) {
    err = hipEventRecord(tm.ev[2 * tm.used + 1], s);
    if (err != hipSuccess) return fail_hip(err, "timing event");
    ++tm.used;
  }
  return PLH_OK;
}

int plh_forward_noalloc(const void* packed_dev, int input_size, int hidden_size, int num_layers, int output_size,
                        const void* x, int batch, int seq_len, const int32_t* lengths, const void* h0, const void* c0,
                        void* out, void* out_seq, void* h_n, void* c_n, const int32_t* probe_steps, int n_probe,
                        float* probe_h, float* probe_c, void* stream) {
  if (batch < 0 || seq_len < 0) return fail(PLH_ERR_INVALID, "batch and seq_len must be non-negative");
  const int64_t need = plh_workspace_bytes(input_size, hidden_size, num_layers, output_size, batch, seq_len);
  if (need < 0) return geometry_code(input_size, hidden_size, num_layers, output_size);
  if ((uint64_t)need > kScratchBytes)
    return fail(PLH_ERR_INVALID, "plh_forward_noalloc: this forward needs " + std::to_string(need) +
                                     " bytes of workspace, more than the " + std::to_string(kScratchBytes >> 20) +
                                     " MiB of device scratch it holds (use plh_forward with a workspace)");
  hipError_t err = hipSuccess;
  void* ws = scratch_ptr(&err);
  if (!ws) return fail_hip(err, "scratch symbol lookup");
  return plh_forward(packed_dev, input_size, hidden_size, num_layers, output_size, x, batch, seq_len, lengths, h0, c0,
                     out, out_seq, h_n, c_n, probe_steps, n_probe, probe_h, probe_c, ws, (int64_t)kScratchBytes,
                     stream);
}

int64_t plh_noalloc_scratch_bytes(void) { return (int64_t)kScratchBytes; }

int plh_noalloc_status(uint32_t* status, void* stream) {
  if (!status) return fail(PLH_ERR_INVALID, "status is required");
  hipError_t err = hipSuccess;
  void* ws = scratch_ptr(&err);
  if (!ws) return fail_hip(err, "scratch symbol lookup");
  return plh_status(ws, status, stream);  // the status word opens the workspace plh_forward lays out there
}

int plh_kernel_timing(int max_forwards) {
  KernelTiming& tm = timing();
  if (max_forwards < 0) {
    tm.release();
    return fail(PLH_ERR_INVALID, "max_forwards must be non-negative");
  }
  if (max_forwards > 0 && (int)tm.ev.size() == 2 * max_forwards) {
    tm.used = 0;  // the same count again: re-arm the events already made (no HIP call)
    return PLH_OK;
  }
  tm.release();
  for (int i = 0; i < 2 * max_forwards; ++i) {
    hipEvent_t e;
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) {
      tm.release();
      return fail_hip(err, "timing event creation");
    }
    tm.ev.push_back(e);
  }
  return PLH_OK;
}

int plh_kernel_timing_read(double* total_ms, int* forwards) {
  if (!total_ms || !forwards) return fail(PLH_ERR_INVALID, "total_ms and forwards are required");
  KernelTiming& tm = timing();
  double sum = 0.0;
  for (int i = 0; i < tm.used; ++i) {
    float ms = 0.0f;
    hipError_t err = hipEventSynchronize(tm.ev[2 * i + 1]);
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, tm.ev[2 * i], tm.ev[2 * i + 1]);
    if (err != hipSuccess) return fail_hip(err, "timing read");
    sum += ms;
  }
  *total_ms = sum;
  *forwards = tm.used;
  return PLH_OK;
}

int plh_input_projection(const void* x, int64_t ldx, const void* w, int k, void* out, int64_t ldo, int64_t rows,
                         int cols, int blocked, void* stream) {
  if (blocked != 0 && blocked != 1) return fail(PLH_ERR_INVALID, "blocked must be 0 or 1");
  if (!plh::gemm_shape_ok(rows, cols, k, ldx, ldo, blocked != 0))
    return fail(PLH_ERR_INVALID, "plh_input_projection needs rows >= 0, cols % 128 == 0, k % 128 == 0, "
                                 "k <= 65536, ldx >= k and ldo >= cols (multiples of 8; blocked: of 32, "
                                 "rows % 16 == 0)");
  if (rows > 0 && (!x || !w || !out)) return fail(PLH_ERR_INVALID, "x, w and out are required");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(out, 16))
    return fail(PLH_ERR_INVALID, "x, w and out must be 16-byte aligned");
  hipError_t err = hipSuccess;
  const int cus = device_cus(&err);
  if (err != hipSuccess) return fail_hip(err, "device query");
  err = plh::launch_proj_gemm((const _Float16*)x, ldx, (const _Float16*)w, k, (_Float16*)out, ldo, rows, cols,
                              blocked != 0, cus, (hipStream_t)stream);
  if (err != hipSuccess) return fail_hip(err, "input projection GEMM launch");
  return PLH_OK;
}

int plh_status(const void* workspace, uint32_t* status, void* stream) {
  if (!workspace || !status) return fail(PLH_ERR_INVALID, "workspace and status are required");
  hipError_t e = hipMemcpyAsync(status, workspace, sizeof(uint32_t), hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "status read");
  return PLH_OK;
}

int plh_set_wait_limit_us(int64_t limit_us) {
  g_wait_us = limit_us > 0 ? limit_us : kDefaultWaitUs;
  return PLH_OK;
}

int plh_inject_wait_failure(int step) {
  g_fail_step = step >= 0 ? step : -1;
  return PLH_OK;
}

int plh_repeat_first_row(const void* in, void* out, int rows, int cols, void* stream) {
  if (rows < 0 || cols < 0) return fail(PLH_ERR_INVALID, "rows and cols must be non-negative");
  if ((rows > 0 && cols > 0) && (!in || !out)) return fail(PLH_ERR_INVALID, "in and out are required");
  hipError_t e = plh::launch_repeat_first_row((const _Float16*)in, (_Float16*)out, rows, cols, (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "repeat_first_row launch");
  return PLH_OK;
}

int plh_probe_mfma_f16(double* tflops, double* clock_ghz) {
  if (!tflops || !clock_ghz) return fail(PLH_ERR_INVALID, "tflops and clock_ghz are required");
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return fail_hip(e, "probe device query");
  // One workgroup of 16 waves per CU (four waves per SIMD); about 15 ms per launch.
  const int blocks = cus, iters = 65536;
  float* out = nullptr;
  unsigned long long* clk = nullptr;
  hipEvent_t ev[2] = {nullptr, nullptr};
  std::vector<unsigned long long> h((size_t)2 * blocks);
  float ms = 0.f;
  e = hipMalloc(&out, (size_t)blocks * 1024 * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&clk, h.size() * sizeof(unsigned long long));
  if (e == hipSuccess) e = hipEventCreate(&ev[0]);
  if (e == hipSuccess) e = hipEventCreate(&ev[1]);
  if (e == hipSuccess) e = plh::launch_mfma_probe(blocks, iters, out, clk, nullptr);  // warm-up (clocks ramp)
  if (e == hipSuccess) e = hipEventRecord(ev[0], nullptr);
  if (e == hipSuccess) e = plh::launch_mfma_probe(blocks, iters, out, clk, nullptr);
  if (e == hipSuccess) e = hipEventRecord(ev[1], nullptr);
  if (e == hipSuccess) e = hipEventSynchronize(ev[1]);
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[0], ev[1]);
  if (e == hipSuccess) e = hipMemcpy(h.data(), clk, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  for (hipEvent_t x : ev)
    if (x) (void)hipEventDestroy(x);
  if (out) (void)hipFree(out);
  if (clk) (void)hipFree(clk);
  if (e != hipSuccess) return fail_hip(e, "MFMA probe");
  double cycles = 0.0, ticks = 0.0;
  for (int b = 0; b < blocks; ++b) {
    cycles += (double)h[2 * b];
    ticks += (double)h[2 * b + 1];
  }
  *tflops = ms > 0.f ? plh::mfma_probe_flops(blocks, iters) / (ms * 1e-3) / 1e12 : 0.0;
  *clock_ghz = ticks > 0.0 ? cycles / (ticks * 10.0) : 0.0;  // 100 MHz ticks: 10 ns each
  return PLH_OK;
}

}  // extern "C"
