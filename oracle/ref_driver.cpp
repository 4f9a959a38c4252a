// ref_driver.cpp -- a C entry point around the reference's own CPU path (test infrastructure only).
//
// It wraps raw float32 buffers as ATen tensors and calls persistent_lstm4_forward_reference
// (persistent_lstm_hip/csrc/persistent_lstm_reference.cpp:42-64), which is compiled, unmodified,
// from where it lies in the reference checkout.  Used as the checker of the C oracle and as the
// CPU baseline (kind "reference"); never by the product path.
#include <ATen/Parallel.h>
#include <torch/torch.h>

#include <cstdint>
#include <cstring>

torch::Tensor persistent_lstm4_forward_reference(
    const torch::Tensor& x, const torch::Tensor& weight_ih_l0, const torch::Tensor& weight_hh_l0,
    const torch::Tensor& bias_l0, const torch::Tensor& weight_ih_l1, const torch::Tensor& weight_hh_l1,
    const torch::Tensor& bias_l1, const torch::Tensor& weight_ih_l2, const torch::Tensor& weight_hh_l2,
    const torch::Tensor& bias_l2, const torch::Tensor& weight_ih_l3, const torch::Tensor& weight_hh_l3,
    const torch::Tensor& bias_l3, const torch::Tensor& linear_weight, const torch::Tensor& linear_bias);

namespace {
torch::Tensor wrap(const float* p, std::initializer_list<int64_t> shape) {
  return torch::from_blob(const_cast<float*>(p), shape, torch::TensorOptions().dtype(torch::kFloat32));
}
}  // namespace

// x [B,T,I]; w_ih[l] [4H,K_l]; w_hh[l] [4H,H]; bias[l] [4H] (already b_ih + b_hh);
// w_lin [O,H]; b_lin [O]; out [B,O].  threads <= 0 keeps ATen's default.  Returns 0 on success.
extern "C" int ref_lstm4_forward(int B, int T, int I, int H, int O, const float* x,
                                 const float* const* w_ih, const float* const* w_hh,
                                 const float* const* bias, const float* w_lin, const float* b_lin,
                                 float* out, int threads) {
  try {
    if (threads > 0) at::set_num_threads(threads);
    auto xt = wrap(x, {B, T, I});
    torch::Tensor wi[4], wh[4], bb[4];
    for (int l = 0; l < 4; ++l) {
      wi[l] = wrap(w_ih[l], {4 * H, l == 0 ? I : H});
      wh[l] = wrap(w_hh[l], {4 * H, H});
      bb[l] = wrap(bias[l], {4 * H});
    }
    auto y = persistent_lstm4_forward_reference(xt, wi[0], wh[0], bb[0], wi[1], wh[1], bb[1], wi[2],
                                                wh[2], bb[2], wi[3], wh[3], bb[3],
                                                wrap(w_lin, {O, H}), wrap(b_lin, {O}))
                 .contiguous();
    std::memcpy(out, y.data_ptr<float>(), sizeof(float) * (size_t)B * O);
    return 0;
  } catch (...) {
    return -1;
  }
}

extern "C" int ref_num_threads(void) { return at::get_num_threads(); }
