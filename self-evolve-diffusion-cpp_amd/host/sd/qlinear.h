// GPU int8 Linear for the DiT blocks: the device side of the reference's
// `mlin` (src/model/ovi_dit.cpp:66-84) and of the consumers that follow it.
//
// A QLinear is built once from the I8 [out,in] view + ".scale" view that
// load_sdcpp returns (checked to sit right after the int8 blob, as
// OviDit::load_impl's lin() requires, ovi_dit.cpp:397-415) and an F32 bias.
// Host-tensor calls (mlin*) are synchronous and bit-identical to the
// reference's qgemm + bias pass (+ gated_add_inplace / add_inplace);
// device-pointer calls (forward_device) are stream-ordered.
#pragma once
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "sd/tensor.h"
#include "sdq.h"

namespace sd {
namespace gpu {

// One [out,in] int8 Linear's arrays (all host or all device memory).
struct LinearPart {
  const int8_t* w = nullptr;     // [out,in] row-major
  const float* scale = nullptr;  // [out], may be unaligned (.sdcpp v1)
  const float* bias = nullptr;   // [out] or nullptr
  int64_t out = 0, in = 0;
};

// One [out,in] int8 Linear inside a .sdcpp file: absolute offsets of its
// int8 rows and scales (sd::PackEntry), and its bias already read (host).
struct FilePart {
  uint64_t q_off = 0, scale_off = 0;
  std::vector<float> bias;  // [out] or empty
  int64_t out = 0, in = 0;
};

class QLinear {
 public:
  QLinear() = default;
  // w: I8 [out,in] view; scale: F32 [out] view; bias: F32 [out] or empty.
  QLinear(const Tensor& w, const Tensor& scale, const Tensor& bias);
  // Several Linears that read the same input, concatenated along out (one
  // weight [sum out, in]): bit-identical to running them separately, since
  // activations are quantized per row and each output column depends only
  // on its own weight row and scale. Parts in host memory, or in device
  // memory with on_device (then the concatenation and repack stay on the GPU).
  explicit QLinear(const std::vector<LinearPart>& parts, bool on_device = false);
  // Many Linears (each one or more parts, host arrays) in one streamed upload
  // (sdq_weight_upload_batch: pinned staging, async copies, repack overlap).
  static std::vector<QLinear> upload_many(const std::vector<std::vector<LinearPart>>& linears);
  // The same straight from a pack file with sequential reads
  // (sdq_weight_upload_file): no page faults through a mapping.
  static std::vector<QLinear> upload_many_file(const std::string& path,
                                               const std::vector<std::vector<FilePart>>& linears);
  QLinear(const QLinear&) = delete;
  QLinear& operator=(const QLinear&) = delete;
  QLinear(QLinear&& o) noexcept;
  QLinear& operator=(QLinear&& o) noexcept;
  ~QLinear();

  int64_t in_features() const { return K_; }
  int64_t out_features() const { return N_; }
  const sdq_weight* handle() const { return w_; }
  const float* bias_device() const { return bias_dev_; }

  // y = x W^T + b    (mlin, ovi_dit.cpp:66-84)
  void mlin(const Tensor& x, Tensor& y) const;
  // y = gelu_tanh(x W^T + b)   (ffn fc1 + gelu_tanh_inplace, ovi_dit.cpp:217-218)
  void mlin_gelu(const Tensor& x, Tensor& y) const;
  // res += (x W^T + b) * gate   (gated_add_inplace, ovi_dit.cpp:152-159, fma form)
  void mlin_gated_add(const Tensor& x, const Tensor& gate, Tensor& res) const;
  // res += x W^T + b   (add_inplace, ovi_dit.cpp:144-149)
  void mlin_add(const Tensor& x, Tensor& res) const;

  // Device pointers, stream-ordered: Y = epilogue(x W^T + b).
  void forward_device(const float* x, int64_t M, int kind, const float* gate, const float* resid,
                      float* Y, void* stream) const;

 private:
  void run_host(const Tensor& x, int kind, const Tensor* gate, Tensor* res, Tensor* y) const;
  void upload_bias(const float* b, bool on_device);
  sdq_weight* w_ = nullptr;
  float* bias_dev_ = nullptr;
  std::vector<float> bias_host_;
  int64_t N_ = 0, K_ = 0;
};

// OviDit::load_impl's lin() (src/model/ovi_dit.cpp:397-415) on a load_sdcpp
// map: "<base>.weight" must be I8 [out,in] with "<base>.weight.scale" stored
// right after the int8 blob, and "<base>.bias" F32 [out]. Throws
// std::runtime_error("ovi_dit: …") like the reference otherwise.
QLinear qlinear_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                          const std::string& base, int64_t in, int64_t out);
// The same checks, returning the views as a LinearPart (host memory).
LinearPart linear_part_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                                 const std::string& base, int64_t in, int64_t out);

// Owning device array of floats (sdq_device_alloc), move-only.
class DeviceFloats {
 public:
  DeviceFloats() = default;
  explicit DeviceFloats(size_t n);
  DeviceFloats(const DeviceFloats&) = delete;
  DeviceFloats& operator=(const DeviceFloats&) = delete;
  DeviceFloats(DeviceFloats&& o) noexcept : p_(o.p_) { o.p_ = nullptr; }
  DeviceFloats& operator=(DeviceFloats&& o) noexcept;
  ~DeviceFloats();
  float* get() const { return p_; }
  explicit operator bool() const { return p_ != nullptr; }

 private:
  float* p_ = nullptr;
};

// mlin (src/model/ovi_dit.cpp:66-84) for either weight dtype a pack holds:
// I8 -> the int8 path (QLinear: qgemm + the bias pass), F32 / BF16 -> the
// fp32 matmul of blk::linear (sdq_linear_f32: one fused multiply-add chain
// per output in k order, then + bias, as sd::matmul computes it,
// src/core/gemm.cpp:115-160). Both branches are bit-exact with the reference.
class Linear {
 public:
  Linear() = default;
  // An fp32 Linear from the torch [out, in] weight (transposed to [in, out]
  // on upload, as lin() does, ovi_dit.cpp:409); bias [out] or nullptr. Host arrays.
  Linear(const float* w_out_in, const float* bias, int64_t out, int64_t in);
  explicit Linear(QLinear&& q);
  Linear(Linear&&) noexcept = default;
  Linear& operator=(Linear&&) noexcept = default;
  bool is_int8() const { return !f32_; }
  const QLinear& int8() const { return q_; }
  int64_t in_features() const { return in_; }
  int64_t out_features() const { return out_; }
  // y = x W^T + b on host tensors (synchronous).
  void mlin(const Tensor& x, Tensor& y) const;
  // Device arrays x [M, in], y [M, out], stream-ordered.
  void forward_device(const float* x, int64_t M, float* y, void* stream) const;

 private:
  QLinear q_;
  DeviceFloats w_, b_;  // fp32 branch: [in, out] weight, bias (or empty)
  int64_t in_ = 0, out_ = 0;
  bool f32_ = false;
};

// OviDit::load_impl's lin() (ovi_dit.cpp:397-415) for either dtype:
// "<base>.weight" [out, in] (I8 with its scale blob right after the int8
// data, or F32 / BF16) and "<base>.bias" [out]; the reference's checks and
// "ovi_dit: …" messages.
Linear linear_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                        const std::string& base, int64_t in, int64_t out);

// Throws std::runtime_error with sdq_last_error() when rc != SDQ_OK.
void check(int rc, const char* what);

}  // namespace gpu
}  // namespace sd
