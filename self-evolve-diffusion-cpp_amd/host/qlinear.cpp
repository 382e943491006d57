// sd::gpu::QLinear — see sd/qlinear.h.
#include "sd/qlinear.h"

#include <stdexcept>
#include <string>
#include <utility>

namespace sd {
namespace gpu {

void check(int rc, const char* what) {
  if (rc != SDQ_OK) throw std::runtime_error(std::string(what) + ": " + sdq_last_error());
}

QLinear::QLinear(const Tensor& w, const Tensor& scale, const Tensor& bias) {
  if (w.dtype != DType::I8 || w.shape.size() != 2)
    throw std::runtime_error("QLinear: weight must be a 2-D I8 [out,in] view");
  N_ = w.rows();
  K_ = w.cols();
  if (scale.dtype != DType::F32 || scale.numel() != N_)
    throw std::runtime_error("QLinear: scale must be F32 [out]");
  if (bias.data && (bias.dtype != DType::F32 || bias.numel() != N_))
    throw std::runtime_error("QLinear: bias must be F32 [out]");
  check(sdq_weight_upload(w.ptr<int8_t>(), scale.ptr<float>(), N_, K_, nullptr, &w_),
        "QLinear: weight upload");
  if (bias.data) {
    bias_host_.assign(bias.ptr<float>(), bias.ptr<float>() + N_);
    void* p = nullptr;
    int rc = sdq_device_alloc((size_t)N_ * 4, &p);
    if (rc == SDQ_OK) rc = sdq_memcpy(p, bias_host_.data(), (size_t)N_ * 4, SDQ_H2D, nullptr);
    if (rc == SDQ_OK) rc = sdq_stream_sync(nullptr);
    if (rc != SDQ_OK) {
      sdq_device_free(p);
      sdq_weight_free(w_);
      w_ = nullptr;
      check(rc, "QLinear: bias upload");
    }
    bias_dev_ = static_cast<float*>(p);
  }
}

QLinear::QLinear(QLinear&& o) noexcept { *this = std::move(o); }

QLinear& QLinear::operator=(QLinear&& o) noexcept {
  if (this != &o) {
    sdq_weight_free(w_);
    sdq_device_free(bias_dev_);
    w_ = o.w_;
    bias_dev_ = o.bias_dev_;
    bias_host_ = std::move(o.bias_host_);
    N_ = o.N_;
    K_ = o.K_;
    o.w_ = nullptr;
    o.bias_dev_ = nullptr;
  }
  return *this;
}

QLinear::~QLinear() {
  sdq_weight_free(w_);
  sdq_device_free(bias_dev_);
}

void QLinear::run_host(const Tensor& x, int kind, const Tensor* gate, Tensor* res,
                       Tensor* y) const {
  if (!w_) throw std::runtime_error("QLinear: empty");
  if (x.dtype != DType::F32) throw std::runtime_error("QLinear: x must be F32");
  const int64_t M = x.rows(), K = x.cols();
  if (K != K_)
    throw std::runtime_error("QLinear: x has " + std::to_string(K) + " columns, weight expects " +
                             std::to_string(K_));
  sdq_epilogue e{};
  e.kind = kind;
  e.gate_fma = 1;
  e.bias = bias_host_.empty() ? nullptr : bias_host_.data();
  if (gate) {
    if (gate->numel() != N_) throw std::runtime_error("QLinear: gate must have out entries");
    e.gate = gate->ptr<float>();
  }
  void* dst;
  if (res) {
    if (res->rows() != M || res->cols() != N_ || res->dtype != DType::F32)
      throw std::runtime_error("QLinear: residual must be F32 [M,out]");
    e.resid = res->ptr<float>();
    dst = res->data;
  } else {
    *y = Tensor({M, N_}, DType::F32);
    dst = y->data;
  }
  check(sdq_qlinear_host(w_, x.ptr<float>(), M, K, &e, dst), "QLinear");
}

void QLinear::mlin(const Tensor& x, Tensor& y) const { run_host(x, SDQ_EPI_NONE, nullptr, nullptr, &y); }

void QLinear::mlin_gelu(const Tensor& x, Tensor& y) const {
  run_host(x, SDQ_EPI_GELU, nullptr, nullptr, &y);
}

void QLinear::mlin_gated_add(const Tensor& x, const Tensor& gate, Tensor& res) const {
  run_host(x, SDQ_EPI_GATED, &gate, &res, nullptr);
}

void QLinear::mlin_add(const Tensor& x, Tensor& res) const {
  run_host(x, SDQ_EPI_RESID, nullptr, &res, nullptr);
}

void QLinear::forward_device(const float* x, int64_t M, int kind, const float* gate,
                             const float* resid, float* Y, void* stream) const {
  sdq_epilogue e{};
  e.kind = kind;
  e.gate_fma = 1;
  e.bias = bias_dev_;
  e.gate = gate;
  e.resid = resid;
  check(sdq_qlinear(w_, x, M, K_, &e, Y, stream), "QLinear::forward_device");
}

QLinear qlinear_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                          const std::string& base, int64_t in, int64_t out) {
  auto get = [&](const std::string& n) -> const Tensor& {
    auto it = pack.find(n);
    if (it == pack.end() || !it->second.data)
      throw std::runtime_error("ovi_dit: missing tensor " + n);
    return it->second;
  };
  const Tensor& w = get(base + ".weight");
  if (w.shape.size() != 2 || w.shape[0] != out || w.shape[1] != in)
    throw std::runtime_error("ovi_dit: bad shape for " + base + ".weight");
  if (w.dtype != DType::I8)
    throw std::runtime_error("ovi_dit: " + base + ".weight is not an int8 pack entry");
  const Tensor& sc = get(base + ".weight.scale");
  if (sc.data != static_cast<const char*>(w.data) + w.numel())
    throw std::runtime_error("ovi_dit: scale not packed after i8 for " + base);
  const Tensor& b = get(base + ".bias");
  if (b.dtype != DType::F32 || b.shape.size() != 1 || b.shape[0] != out)
    throw std::runtime_error("ovi_dit: bad shape for " + base + ".bias");
  return QLinear(w, sc, b);
}

}  // namespace gpu
}  // namespace sd
