/*
 * lstm_oracle.c -- CPU restatement of the reference's stacked LSTM + Linear forward.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it.  The product path (persistent_lstm_hip_amd) never
 * links, loads or calls it, and must fail loudly when its HIP library is missing.
 *
 * What it restates (reference = mantuoluozk/persistent_lstm_hip):
 *   - textbook per-layer recurrence with h0 = c0 = 0, gate order i, f, g, o along the 4H axis:
 *       persistent_lstm_hip/csrc/persistent_lstm_reference.cpp:7-38   (run_layer)
 *       persistent_lstm_hip/persistent_lstm_hip/reference.py:11-63    (reference_lstm_forward)
 *   - 4-layer stack feeding layer l's output sequence into layer l+1:
 *       persistent_lstm_reference.cpp:42-60, reference.py:37-59
 *   - Linear head on the last step of the last layer:
 *       persistent_lstm_reference.cpp:61-63, reference.py:66-72
 *   - optional initial state hx = (h0, c0) of shape [L, B, H]: reference.py:29-32
 *   - "reference device numerics" mode (numerics = 1, and 2 with an fp16 input projection as the
 *     reference's generic path computes it, persistent_lstm_hip.cu:2988-2994) restating the
 *     reference kernels' storage:
 *       bias fused as one fp16 rounding of (b_ih + b_hh)         model.py:552
 *       h rounded to fp16 after every step, c kept in fp32      persistent_lstm_hip.cu:524-525
 *       sigmoid(x) = 1 / (1 + exp(-x)), tanh                   persistent_lstm_hip.cu:96-98
 *       head accumulated in fp32 from fp16 operands, fp16 out  persistent_lstm_hip.cu:1662-1682
 *   - packed-sequence (ragged) semantics, which the reference lacks: row b only processes steps
 *     t < lengths[b]; its state is frozen afterwards and its output sequence is zero there.  This
 *     is torch.nn.utils.rnn.pack_padded_sequence -> nn.LSTM -> pad_packed_sequence semantics.
 *
 * Dot products accumulate in double, so the fp32 mode sits within ~1e-6 of torch's fp32 CPU
 * nn.LSTM; the tests pin it against torch, closed forms and brute-force cases.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- IEEE binary16 conversion, round-to-nearest-even (written from the format definition) ---- */

uint16_t oracle_float_to_half_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t absx = x & 0x7fffffffu;
  if (absx > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* NaN */
  if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf (>= 65520) */
  const int exp = (int)(absx >> 23) - 127;
  uint32_t mant = absx & 0x7fffffu;
  if (exp >= -14) {
    /* normal half: keep 10 mantissa bits, round the dropped 13 bits to nearest even */
    uint32_t h = ((uint32_t)(exp + 15) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry may bump the exponent */
    return (uint16_t)(sign | h);
  }
  if (exp < -25) return (uint16_t)sign; /* below half the smallest subnormal: rounds to zero */
  /* subnormal half: value = m * 2^-24 with m = round(full_mantissa * 2^(exp+24-23)) */
  mant |= 0x800000u;
  const int shift = -exp - 1; /* 14 .. 24: number of bits dropped from the 24-bit significand */
  uint32_t h = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

float oracle_half_bits_to_float(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
  const uint32_t m = (uint32_t)h & 0x3ffu;
  float out;
  if (e == 0) {
    out = ldexpf((float)m, -24);
    if (sign) out = -out;
    return out;
  }
  uint32_t x;
  if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e - 15 + 127) << 23) | (m << 13);
  }
  memcpy(&out, &x, 4);
  return out;
}

float oracle_round_half(float f) { return oracle_half_bits_to_float(oracle_float_to_half_bits(f)); }

void oracle_round_half_array(float* a, int64_t n) {
  for (int64_t i = 0; i < n; ++i) a[i] = oracle_round_half(a[i]);
}

/* ---- activations: sigmoid as in persistent_lstm_hip.cu:96-98, tanh from libm ---- */

static inline double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

/* Planted mistakes, used only by tests to prove that the pins catch them (the oracle's own
 * "mutation testing").  0 = the faithful algorithm. */
enum {
  MUT_NONE = 0,
  MUT_SWAP_IF = 1,         /* read the forget gate where the input gate lives and vice versa */
  MUT_DROP_RECURRENT = 2,  /* forget the h_{t-1} W_hh^T term                                  */
  MUT_TRANSPOSE_WHH = 3,   /* index W_hh as [H, 4H] instead of [4H, H]                        */
  MUT_DROP_BIAS_HH = 4,    /* use only b_ih                                                     */
  MUT_NO_TANH_C = 5,       /* h = o * c instead of o * tanh(c)                                  */
  MUT_GATE_ORDER_IGFO = 6, /* take the gates in i, g, f, o order                                */
};

/*
 * Stacked LSTM forward.  All arrays are row-major float32:
 *   x        [B, T, I]
 *   w_ih[l]  [4H, K_l] (K_0 = I, K_l = H),  w_hh[l] [4H, H],  b_ih[l], b_hh[l] [4H] (b_hh may be NULL)
 *   lengths  [B] int32 or NULL (NULL: every row runs T steps)
 *   h0, c0   [L, B, H] or NULL (zeros)
 *   probe_steps[n_probe]: step counts p in [1, T]; probe_h/probe_c [n_probe, L, B, H] receive the
 *            state after p steps (for ragged rows, after min(p, length) steps)
 *   out_seq  [B, T, H] last layer's output sequence (zero where t >= length), or NULL
 *   h_n, c_n [L, B, H] final states, or NULL
 * numerics: 0 = fp32 textbook, 1 = reference device numerics (see header), 2 = as 1 with the input
 *           projection W_ih x of every step rounded to fp16 before the bias and recurrent terms are
 *           added (the reference's generic path: persistent_lstm_hip.cu:2988-2994 computes it as an
 *           fp16 torch::matmul, the persistent kernel adds the rest in fp32); 3 = as 2 for layers >= 1
 *           only, layer 0's projection kept unrounded (the device's layer-sequential path with
 *           input_size <= 32 computes layer 0's projection in fp32 inside its recurrent kernel).
 * Returns 0, or -1 for invalid arguments.
 */
int oracle_lstm_forward(int B, int T, int I, int H, int L, const float* x, const float* const* w_ih,
                        const float* const* w_hh, const float* const* b_ih, const float* const* b_hh,
                        const int32_t* lengths, const float* h0, const float* c0, int numerics,
                        const int32_t* probe_steps, int n_probe, float* probe_h, float* probe_c,
                        float* out_seq, float* h_n, float* c_n, int mutation, int threads) {
  if (B < 0 || T < 0 || I <= 0 || H <= 0 || L <= 0) return -1;
  if (n_probe > 0 && (!probe_steps || !probe_h || !probe_c)) return -1;
  for (int p = 0; p < n_probe; ++p)
    if (probe_steps[p] < 1 || probe_steps[p] > T) return -1;
  if (lengths)
    for (int b = 0; b < B; ++b)
      if (lengths[b] < 0 || lengths[b] > T) return -1;
  const int G = 4 * H;
  const int Kmax = I > H ? I : H;

  /* fused bias per layer (model.py:552 rounds the fp16 sum once in device-numerics mode) */
  double* bias = (double*)malloc(sizeof(double) * (size_t)L * G);
  if (!bias) return -1;
  for (int l = 0; l < L; ++l)
    for (int g = 0; g < G; ++g) {
      float bh = (b_hh && b_hh[l] && mutation != MUT_DROP_BIAS_HH) ? b_hh[l][g] : 0.0f;
      float bs = b_ih[l] ? b_ih[l][g] : 0.0f;
      bias[(size_t)l * G + g] = numerics ? (double)oracle_round_half(bs + bh) : (double)bs + (double)bh;
    }

#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
#endif
  {
    float* in = (float*)malloc(sizeof(float) * (size_t)T * Kmax);
    float* out = (float*)malloc(sizeof(float) * (size_t)T * H);
    double* acc = (double*)malloc(sizeof(double) * G);
    float* h = (float*)malloc(sizeof(float) * H);
    float* c = (float*)malloc(sizeof(float) * H);
    float* hn = (float*)malloc(sizeof(float) * H);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int b = 0; b < B; ++b) {
      const int len = lengths ? lengths[b] : T;
      for (int t = 0; t < T; ++t)
        for (int k = 0; k < I; ++k) in[(size_t)t * Kmax + k] = x[((size_t)b * T + t) * I + k];
      int K = I;
      for (int l = 0; l < L; ++l) {
        const float* Wi = w_ih[l];
        const float* Wh = w_hh[l];
        const double* bl = bias + (size_t)l * G;
        for (int u = 0; u < H; ++u) {
          h[u] = h0 ? h0[((size_t)l * B + b) * H + u] : 0.0f;
          c[u] = c0 ? c0[((size_t)l * B + b) * H + u] : 0.0f;
          if (numerics) h[u] = oracle_round_half(h[u]);
        }
        for (int t = 0; t < T; ++t) {
          if (t < len) {
            for (int g = 0; g < G; ++g) {
              const float* wi = Wi + (size_t)g * K;
              const float* xt = in + (size_t)t * Kmax;
              double p = 0.0;
              for (int k = 0; k < K; ++k) p += (double)wi[k] * (double)xt[k];
              /* numerics 2: the input projection is an fp16 tensor (the reference's generic path,
                 torch::matmul of fp16 operands, persistent_lstm_hip.cu:2988-2994) */
              if (numerics == 2 || (numerics == 3 && l > 0)) p = (double)oracle_round_half((float)p);
              double a = bl[g] + p;
              if (mutation != MUT_DROP_RECURRENT) {
                if (mutation == MUT_TRANSPOSE_WHH) {
                  for (int j = 0; j < H; ++j) a += (double)Wh[(size_t)j * G + g] * (double)h[j];
                } else {
                  const float* wh = Wh + (size_t)g * H;
                  for (int j = 0; j < H; ++j) a += (double)wh[j] * (double)h[j];
                }
              }
              acc[g] = a;
            }
            int gi = 0, gf = 1, gg = 2, go = 3;
            if (mutation == MUT_SWAP_IF) { gi = 1; gf = 0; }
            if (mutation == MUT_GATE_ORDER_IGFO) { gg = 1; gf = 2; }
            for (int u = 0; u < H; ++u) {
              const double ig = sigmoid_d(acc[gi * H + u]);
              const double fg = sigmoid_d(acc[gf * H + u]);
              const double g_ = tanh(acc[gg * H + u]);
              const double og = sigmoid_d(acc[go * H + u]);
              const double cn = fg * (double)c[u] + ig * g_;
              c[u] = (float)cn;
              const double hv = (mutation == MUT_NO_TANH_C) ? og * cn : og * tanh(cn);
              hn[u] = numerics ? oracle_round_half((float)hv) : (float)hv;
            }
            memcpy(h, hn, sizeof(float) * H);
            memcpy(out + (size_t)t * H, h, sizeof(float) * H);
          } else {
            memset(out + (size_t)t * H, 0, sizeof(float) * H);
          }
          for (int p = 0; p < n_probe; ++p) {
            if (probe_steps[p] == t + 1) {
              const size_t o = (((size_t)p * L + l) * B + b) * H;
              memcpy(probe_h + o, h, sizeof(float) * H);
              memcpy(probe_c + o, c, sizeof(float) * H);
            }
          }
        }
        if (h_n) memcpy(h_n + ((size_t)l * B + b) * H, h, sizeof(float) * H);
        if (c_n) memcpy(c_n + ((size_t)l * B + b) * H, c, sizeof(float) * H);
        /* this layer's output sequence is the next layer's input (reference.py:59) */
        for (int t = 0; t < T; ++t) memcpy(in + (size_t)t * Kmax, out + (size_t)t * H, sizeof(float) * H);
        K = H;
      }
      if (out_seq)
        for (int t = 0; t < T; ++t)
          memcpy(out_seq + ((size_t)b * T + t) * H, in + (size_t)t * Kmax, sizeof(float) * H);
    }
    free(in);
    free(out);
    free(acc);
    free(h);
    free(c);
    free(hn);
  }
  free(bias);
  return 0;
}

/*
 * Linear head: out[b, o] = bias[o] + sum_k in[b, k] * w[o, k]   (reference.py:72, cu:1662-1682).
 * numerics = 1 rounds the result to fp16 as the reference's head kernel does.
 */
int oracle_linear(int B, int K, int O, const float* in, const float* w, const float* bias, float* out,
                  int numerics) {
  if (B < 0 || K <= 0 || O <= 0) return -1;
  for (int b = 0; b < B; ++b)
    for (int o = 0; o < O; ++o) {
      double a = bias ? (double)bias[o] : 0.0;
      for (int k = 0; k < K; ++k) a += (double)in[(size_t)b * K + k] * (double)w[(size_t)o * K + k];
      out[(size_t)b * O + o] = numerics ? oracle_round_half((float)a) : (float)a;
    }
  return 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
