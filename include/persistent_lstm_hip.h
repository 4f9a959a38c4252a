/*
 * persistent_lstm_hip.h -- C ABI of the MI355X (gfx950) stacked LSTM + Linear inference forward.
 *
 * Library: persistent_lstm_hip_amd/lib/libpersistent_lstm_hip.so
 *
 * Conventions
 *   - Every pointer named *_dev, and every tensor argument, is device memory on the current HIP
 *     device.  fp16 tensors are IEEE binary16 (torch.float16), row-major, contiguous.
 *   - `stream` is a hipStream_t (may be NULL for the null stream).  Entry points only enqueue
 *     work on that stream; none of them synchronises except plh_status().
 *   - Return value: PLH_OK, or an error code; plh_last_error() gives the calling thread's message.
 *     PLH_ERR_INVALID and PLH_ERR_UNSUPPORTED correspond to the reference's std::invalid_argument
 *     (Python ValueError, persistent_lstm_op.cpp:7-11); PLH_ERR_HIP to its std::runtime_error with
 *     the hipGetErrorString text (Python RuntimeError, persistent_lstm_hip.cu:1730-1735).
 *   - Model geometry: I = input size, H = hidden size, L = layers, O = Linear output size
 *     (O = 0: no head).  Gate order along the 4H axis is i, f, g, o as in torch.nn.LSTM.
 *   - Numerics: fp16 weights and activations, fp32 MFMA accumulation, c kept in fp32, h rounded
 *     to fp16 every step, fused bias b_ih + b_hh summed in fp32, head accumulated in fp32 and
 *     written as fp16.
 *
 * Reference interface each entry point replaces (mantuoluozk/persistent_lstm_hip):
 *   bindings.cpp:154-165 exports the pybind functions the Python dispatcher calls.  The weight
 *   repacking that model.py:542-582 / :20-27 does on the Python side becomes plh_pack_regressor,
 *   and the family of fixed-shape forwards collapses into plh_forward.
 */
#ifndef PERSISTENT_LSTM_HIP_H
#define PERSISTENT_LSTM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PLH_OK 0
#define PLH_ERR_INVALID 1     /* bad argument (shape, size, null pointer)        -> ValueError   */
#define PLH_ERR_UNSUPPORTED 2 /* geometry outside what the kernels implement      -> ValueError   */
#define PLH_ERR_HIP 3         /* HIP runtime error                                -> RuntimeError */
#define PLH_ERR_DEVICE 4      /* the persistent kernel reported a failure status  -> RuntimeError */

/* Bits of the device status word read by plh_status(). */
#define PLH_STATUS_TIMEOUT 1u /* a layer hand-off wait exceeded its time limit; outputs are NaN */

/* ABI version of this header. */
int plh_abi_version(void);

/* Message describing the last error raised on the calling thread ("" if none). */
const char* plh_last_error(void);

/* 1 if plh_forward implements this geometry, else 0 (plh_last_error() says why): 1 <= H <= 1024, any
 * input size up to 65536, L <= 64, O <= 4096 (the reference's generic entry point serves
 * 1 <= H <= 1024 and any input size, model.py:154-165, persistent_lstm_hip.cu:2981-2991).
 * Replaces the shape predicates PersistentLSTMRegressor._can_use_specialized_regressor_hip
 * (model.py:432-441) and NativeModuleFallback._can_use_generic_projected_module (model.py:131-165). */
int plh_supports(int input_size, int hidden_size, int num_layers, int output_size);

/* Bytes of the packed-weight blob for a geometry (negative on invalid geometry). */
int64_t plh_packed_bytes(int input_size, int hidden_size, int num_layers, int output_size);

/*
 * Pack torch-layout fp16 parameters into the kernel's resident-weight layout.
 *   w_ih[l]: weight_ih_l{l} [4H, l == 0 ? I : H]      w_hh[l]: weight_hh_l{l} [4H, H]
 *   b_ih[l], b_hh[l]: [4H] (b_hh[l] or the whole b_hh array may be NULL: treated as zero, which also
 *                     lets a caller pass the reference's pre-fused bias b_ih + b_hh in b_ih)
 *   lin_w [O, H], lin_b [O] (ignored when O == 0)
 * w_ih, w_hh, b_ih, b_hh are HOST arrays of L device pointers.
 * Replaces the repack cache fill of model.py:542-582 (kpairs packing, model.py:20-27) and the
 * per-call weight handling of persistent_lstm_regressor_forward_generic_projected_hip
 * (persistent_lstm_hip.cu:2923-3000).
 */
int plh_pack_regressor(int input_size, int hidden_size, int num_layers, int output_size,
                       const void* const* w_ih, const void* const* w_hh, const void* const* b_ih,
                       const void* const* b_hh, const void* lin_w, const void* lin_b,
                       void* packed_dev, int64_t packed_bytes, void* stream);

/* Bytes of device workspace plh_forward needs for (geometry, batch, seq_len).  At padded H 512 it
 * depends on the path the launch plan picks for that batch and length (the layer-sequential one
 * holds a layer's input projection for every step: about 3 MB per step at 512 rows). */
int64_t plh_workspace_bytes(int input_size, int hidden_size, int num_layers, int output_size, int batch,
                            int seq_len);

/*
 * Stacked LSTM (+ optional Linear head) forward over x [batch, seq_len, I] fp16 (batch_first).
 *   lengths   device int32 [batch] or NULL.  NULL: every row runs seq_len steps.  Otherwise
 *             packed-sequence semantics: row b runs lengths[b] steps, its state is frozen after,
 *             out_seq is zero past its length and the head reads its state at its last step.
 *   h0, c0    device fp16 [L, batch, H] initial state, or NULL for zeros (nn.LSTM hx).
 *   out       device fp16 [batch, O]: Linear(h_n[L-1]) (= Linear(out_seq[:, -1]) for full rows).
 *   out_seq   device fp16 [batch, seq_len, H]: last layer's outputs, or NULL.
 *   h_n, c_n  device fp16 [L, batch, H] final states, or NULL.
 *   probe_steps device int32 [n_probe], strictly increasing step counts in [1, seq_len];
 *             probe_h / probe_c device fp32 [n_probe, L, batch, H] receive every layer's state
 *             after that many steps (h as rounded to fp16, c in fp32).  n_probe = 0: no probes.
 *   workspace device memory of at least plh_workspace_bytes(...) bytes, 256-byte aligned.
 * Any output pointer may be NULL.  Asynchronous on `stream`; forwards on different streams of one
 * device are ordered by the library (each needs the whole device co-resident): the first forward
 * on a second stream synchronises the device once, later ones wait on an event of the previous
 * forward when it was on another stream (not inside a stream capture).  Hidden sizes 513..1024, inputs wider
 * than the padded hidden size, and at padded H 512 a batch that needs more wavefront launches than
 * there are layers run layer by layer: per layer the input projection of every step as one fp16
 * MFMA GEMM (plh_input_projection's kernel; for layer 0 with input_size <= 32 at H > 256 inside the
 * recurrent kernel), then a W_hh-only persistent kernel.  That path rounds the GEMM's x_t W_ih^T to
 * fp16 before the recurrent sum, as the reference's generic path does (persistent_lstm_hip.cu:
 * 2988-2994); the all-layers path keeps it in fp32, so at padded H 512 the batch size decides which
 * of the two roundings a row gets (both are within the tolerance).
 * Replaces persistent_lstm4_forward_interleaved (bindings.cpp:157, persistent_lstm_hip.cu:2126-2254)
 * and persistent_lstm_regressor_forward_generic_projected (bindings.cpp:163,
 * persistent_lstm_hip.cu:2923-3181), whose signatures return only the [batch, O] head output;
 * the state/sequence/probe outputs serve the nn.LSTM drop-in (model.py:323-395) and drift checks.
 */
int plh_forward(const void* packed_dev, int input_size, int hidden_size, int num_layers, int output_size,
                const void* x, int batch, int seq_len, const int32_t* lengths, const void* h0,
                const void* c0, void* out, void* out_seq, void* h_n, void* c_n,
                const int32_t* probe_steps, int n_probe, float* probe_h, float* probe_c, void* workspace,
                int64_t workspace_bytes, void* stream);

/*
 * Time-parallel input projection: out[m][n] = sum_{j < k} x[m][j] * w[n][j] for m < rows, n < cols,
 * fp16 operands and result, fp32 accumulation (MFMA), e.g. one layer's x_t W_ih^T for all T steps
 * of a batch at once (rows = T * batch).
 *   w   device fp16 [cols][k] row-major
 *   blocked = 0: x device fp16 [rows][ldx], out [rows][ldo], row-major
 *   blocked = 1: x and out fragment-blocked, [rows / 16][ld / 32][64][8] halfs: element (r, c) at
 *            (((r / 16) * (ld / 32) + c / 32) * 64 + ((c % 32) / 8) * 16 + r % 16) * 8 + c % 8, so that
 *            every 16 rows x 32 columns are one contiguous 1 KB block (the layout of the
 *            layer-sequential path's layer inputs and projections; the faster form)
 * Requires k % 128 == 0, k <= 65536, cols % 128 == 0, ldx >= k and ldo >= cols multiples of 8
 * (blocked: of 32, and rows % 16 == 0), 16-byte aligned pointers (PLH_ERR_INVALID otherwise;
 * zero-pad K to meet them).  Asynchronous on `stream`.
 * Replaces the reference's torch::matmul input projections of fp16 tensors (the generic path's
 * x.matmul(W_ih^T), persistent_lstm_hip.cu:2988-2994; the projected path's, :2329-2379).
 */
int plh_input_projection(const void* x, int64_t ldx, const void* w, int k, void* out, int64_t ldo, int64_t rows,
                         int cols, int blocked, void* stream);

/*
 * plh_forward without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid allocation).  It uses a device
 * scratch array inside the library, PLH_NOALLOC_SCRATCH_BYTES (64 MiB, plh_noalloc_scratch_bytes()),
 * one per GPU, held until the process ends; it calls no allocating routine.  A forward whose
 * plh_workspace_bytes(...) exceeds it is rejected with PLH_ERR_INVALID before anything is enqueued
 * (e.g. the C2 shape fits up to about 64 rows at 1000 steps).  All calls on one GPU share its scratch:
 * calls that overlap on one GPU (different streams or threads) race; calls ordered on one stream do
 * not.  Everything the kernels read from the scratch is written or cleared by the same call.
 * No counterpart in the reference; outputs and arguments as plh_forward.
 */
#define PLH_NOALLOC_SCRATCH_BYTES ((int64_t)64 << 20)
int plh_forward_noalloc(const void* packed_dev, int input_size, int hidden_size, int num_layers, int output_size,
                        const void* x, int batch, int seq_len, const int32_t* lengths, const void* h0,
                        const void* c0, void* out, void* out_seq, void* h_n, void* c_n,
                        const int32_t* probe_steps, int n_probe, float* probe_h, float* probe_c, void* stream);
int64_t plh_noalloc_scratch_bytes(void);
/* plh_status for plh_forward_noalloc: synchronise `stream` and read the status word the last
 * plh_forward_noalloc on the current device left in its scratch (0 = success, else PLH_STATUS_*
 * bits).  Like the scratch, shared by every caller on that device.  No counterpart in the reference. */
int plh_noalloc_status(uint32_t* status, void* stream);

/* Synchronise `stream` and read the status word the last plh_forward left in `workspace`
 * (0 = success, else PLH_STATUS_* bits).  Returns PLH_OK or PLH_ERR_HIP. */
int plh_status(const void* workspace, uint32_t* status, void* stream);

/*
 * Optional timing of the persistent kernel alone (for benchmarks and profilers of the caller).
 * plh_kernel_timing(n) with n > 0 arms n pairs of HIP events for the calling thread: each later
 * plh_forward on this thread records one pair around its persistent launch(es) (on the
 * layer-sequential H512 path: around all its projection GEMMs and launches), until the n pairs
 * are used.  plh_kernel_timing(0) disarms.  Called again with the n it was armed with, it re-arms
 * the same events without creating any (no HIP call: a caller can arm before its warm-ups and
 * re-arm right before its timed forwards).  plh_kernel_timing_read synchronises on the recorded
 * events and returns the summed elapsed milliseconds and the number of timed forwards.
 * No counterpart in the reference (it only timed whole forwards from Python, LSTM-hip.py:80-91).
 */
int plh_kernel_timing(int max_forwards);
int plh_kernel_timing_read(double* total_ms, int* forwards);

/*
 * Bound on every wait between workgroups of the calling thread's later plh_forward calls, in
 * microseconds (default 2000000; limit_us <= 0 restores the default).  A wait that exceeds it sets
 * PLH_STATUS_TIMEOUT, fails every other wait of the launch and poisons the outputs with NaN, so
 * the kernel always ends.  Failure detection for hung co-resident workgroups; no counterpart in the
 * reference (its kernels spin without bound).
 */
int plh_set_wait_limit_us(int64_t limit_us);

/*
 * Failure injection for tests of the failure path: with step >= 0, the calling thread's later
 * plh_forward calls that run the layer-sequential path make one workgroup of each launch treat its
 * exchange wait at that step as timed out (PLH_STATUS_TIMEOUT, outputs NaN where not computed, every
 * kernel still ends normally).  step < 0 turns it off.  The other paths' first hand-off wait can be
 * made to time out with a small plh_set_wait_limit_us; this path's per-step waits finish too fast
 * for that.  No counterpart in the reference.
 */
int plh_inject_wait_failure(int step);

/* out[r, c] = in[0, c] for r < rows (fp16).  Replaces repeat_first_row
 * (bindings.cpp:164, persistent_lstm_hip.cu:1684-1695, :1784-1809). */
int plh_repeat_first_row(const void* in, void* out, int rows, int cols, void* stream);

/*
 * Diagnostic for benchmarks: the dense fp16 MFMA rate this GPU sustains with
 * v_mfma_f32_16x16x32_f16 (the recurrent kernels' instruction) on every CU, in TFLOP/s, and the
 * shader clock during that run, in GHz (about 30 ms on the current device and the null stream;
 * allocates and frees its own buffers).  No counterpart in the reference, which quotes no peak.
 */
int plh_probe_mfma_f16(double* tflops, double* clock_ghz);

#ifdef __cplusplus
}
#endif

#endif /* PERSISTENT_LSTM_HIP_H */
