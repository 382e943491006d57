// sd::gpu::QLinear — see sd/qlinear.h.
#include "sd/qlinear.h"

#include <algorithm>
#include <cstring>
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
  if (bias.data) upload_bias(bias.ptr<float>(), false);
}

void QLinear::upload_bias(const float* b, bool on_device) {
  bias_host_.assign((size_t)N_, 0.f);
  void* p = nullptr;
  int rc = sdq_device_alloc((size_t)N_ * 4, &p);
  if (rc == SDQ_OK) {
    if (on_device) {
      rc = sdq_memcpy(bias_host_.data(), b, (size_t)N_ * 4, SDQ_D2H, nullptr);
      if (rc == SDQ_OK) rc = sdq_memcpy(p, b, (size_t)N_ * 4, SDQ_D2D, nullptr);
    } else {
      bias_host_.assign(b, b + N_);
      rc = sdq_memcpy(p, bias_host_.data(), (size_t)N_ * 4, SDQ_H2D, nullptr);
    }
  }
  if (rc == SDQ_OK) rc = sdq_stream_sync(nullptr);
  if (rc != SDQ_OK) {
    sdq_device_free(p);
    sdq_weight_free(w_);
    w_ = nullptr;
    check(rc, "QLinear: bias upload");
  }
  bias_dev_ = static_cast<float*>(p);
}

std::vector<QLinear> QLinear::upload_many(const std::vector<std::vector<LinearPart>>& linears) {
  std::vector<sdq_weight_src> src(linears.size());
  for (size_t i = 0; i < linears.size(); i++) {
    const std::vector<LinearPart>& parts = linears[i];
    if (parts.empty() || parts.size() > 4)
      throw std::runtime_error("QLinear::upload_many: 1-4 parts per Linear");
    sdq_weight_src& w = src[i];
    w = sdq_weight_src{};
    w.nparts = (int)parts.size();
    w.K = parts[0].in;
    bool any_bias = false, all_bias = true;
    for (size_t p = 0; p < parts.size(); p++) {
      if (!parts[p].w || !parts[p].scale || parts[p].out <= 0 || parts[p].in != w.K)
        throw std::runtime_error("QLinear: parts must share in_features and have weights");
      w.q[p] = parts[p].w;
      w.scale[p] = parts[p].scale;
      w.rows[p] = parts[p].out;
      any_bias = any_bias || parts[p].bias;
      all_bias = all_bias && parts[p].bias;
    }
    if (any_bias && !all_bias) throw std::runtime_error("QLinear: bias on some parts only");
  }
  std::vector<sdq_weight*> handles(linears.size(), nullptr);
  check(sdq_weight_upload_batch(src.data(), (int)src.size(), nullptr, handles.data()),
        "QLinear::upload_many");
  std::vector<QLinear> out(linears.size());
  for (size_t i = 0; i < linears.size(); i++) {  // each takes its handle first (freed on throw)
    out[i].w_ = handles[i];
    out[i].K_ = src[i].K;
    for (const LinearPart& p : linears[i]) out[i].N_ += p.out;
  }
  for (size_t i = 0; i < linears.size(); i++) {
    if (!linears[i][0].bias) continue;
    std::vector<float> b((size_t)out[i].N_);
    size_t r = 0;
    for (const LinearPart& p : linears[i]) {
      std::memcpy(b.data() + r, p.bias, (size_t)p.out * 4);
      r += (size_t)p.out;
    }
    out[i].upload_bias(b.data(), false);
  }
  return out;
}

std::vector<QLinear> QLinear::upload_many_file(const std::string& path,
                                               const std::vector<std::vector<FilePart>>& linears) {
  std::vector<sdq_weight_fsrc> src(linears.size());
  for (size_t i = 0; i < linears.size(); i++) {
    const std::vector<FilePart>& parts = linears[i];
    if (parts.empty() || parts.size() > 4)
      throw std::runtime_error("QLinear::upload_many_file: 1-4 parts per Linear");
    sdq_weight_fsrc& w = src[i];
    w = sdq_weight_fsrc{};
    w.nparts = (int)parts.size();
    w.K = parts[0].in;
    for (size_t p = 0; p < parts.size(); p++) {
      if (parts[p].out <= 0 || parts[p].in != w.K)
        throw std::runtime_error("QLinear: parts must share in_features");
      if (parts[p].bias.empty() != parts[0].bias.empty())
        throw std::runtime_error("QLinear: bias on some parts only");
      w.q_off[p] = parts[p].q_off;
      w.scale_off[p] = parts[p].scale_off;
      w.rows[p] = parts[p].out;
    }
  }
  std::vector<sdq_weight*> handles(linears.size(), nullptr);
  check(sdq_weight_upload_file(path.c_str(), src.data(), (int)src.size(), nullptr, handles.data()),
        "QLinear::upload_many_file");
  std::vector<QLinear> out(linears.size());
  for (size_t i = 0; i < linears.size(); i++) {  // each takes its handle first (freed on throw)
    out[i].w_ = handles[i];
    out[i].K_ = src[i].K;
    for (const FilePart& p : linears[i]) out[i].N_ += p.out;
  }
  for (size_t i = 0; i < linears.size(); i++) {
    if (linears[i][0].bias.empty()) continue;
    std::vector<float> b;
    b.reserve((size_t)out[i].N_);
    for (const FilePart& p : linears[i]) b.insert(b.end(), p.bias.begin(), p.bias.end());
    out[i].upload_bias(b.data(), false);
  }
  return out;
}

QLinear::QLinear(const std::vector<LinearPart>& parts, bool on_device) {
  if (parts.empty()) throw std::runtime_error("QLinear: no parts");
  K_ = parts[0].in;
  N_ = 0;
  bool any_bias = false, all_bias = true;
  for (const LinearPart& p : parts) {
    if (!p.w || !p.scale || p.out <= 0 || p.in != K_)
      throw std::runtime_error("QLinear: parts must share in_features and have weights");
    N_ += p.out;
    any_bias = any_bias || p.bias;
    all_bias = all_bias && p.bias;
  }
  if (any_bias && !all_bias) throw std::runtime_error("QLinear: bias on some parts only");
  const size_t wbytes = (size_t)N_ * (size_t)K_;
  if (!on_device) {
    std::vector<int8_t> w(wbytes);
    std::vector<float> sc((size_t)N_), b(any_bias ? (size_t)N_ : 0);
    size_t r = 0;
    for (const LinearPart& p : parts) {
      std::memcpy(w.data() + r * K_, p.w, (size_t)p.out * K_);
      std::memcpy(sc.data() + r, p.scale, (size_t)p.out * 4);
      if (any_bias) std::memcpy(b.data() + r, p.bias, (size_t)p.out * 4);
      r += (size_t)p.out;
    }
    check(sdq_weight_upload(w.data(), sc.data(), N_, K_, nullptr, &w_), "QLinear: weight upload");
    if (any_bias) upload_bias(b.data(), false);
    return;
  }
  // device parts: concatenate into temporaries, repack on the GPU
  void *tw = nullptr, *ts = nullptr, *tb = nullptr;
  int rc = sdq_device_alloc(wbytes, &tw);
  if (rc == SDQ_OK) rc = sdq_device_alloc((size_t)N_ * 4, &ts);
  if (rc == SDQ_OK && any_bias) rc = sdq_device_alloc((size_t)N_ * 4, &tb);
  size_t r = 0;
  for (const LinearPart& p : parts) {
    if (rc != SDQ_OK) break;
    rc = sdq_memcpy(static_cast<int8_t*>(tw) + r * K_, p.w, (size_t)p.out * K_, SDQ_D2D, nullptr);
    if (rc == SDQ_OK)
      rc = sdq_memcpy(static_cast<float*>(ts) + r, p.scale, (size_t)p.out * 4, SDQ_D2D, nullptr);
    if (rc == SDQ_OK && any_bias)
      rc = sdq_memcpy(static_cast<float*>(tb) + r, p.bias, (size_t)p.out * 4, SDQ_D2D, nullptr);
    r += (size_t)p.out;
  }
  if (rc == SDQ_OK)
    rc = sdq_weight_upload_device(static_cast<const int8_t*>(tw), static_cast<const float*>(ts),
                                  N_, K_, nullptr, &w_);
  if (rc == SDQ_OK) rc = sdq_stream_sync(nullptr);
  const std::string err = rc == SDQ_OK ? "" : sdq_last_error();
  sdq_device_free(tw);
  sdq_device_free(ts);
  if (rc != SDQ_OK) {
    sdq_device_free(tb);
    sdq_weight_free(w_);
    w_ = nullptr;
    throw std::runtime_error("QLinear: device upload: " + err);
  }
  if (any_bias) {
    try {
      upload_bias(static_cast<const float*>(tb), true);
    } catch (...) {
      sdq_device_free(tb);
      throw;
    }
  }
  sdq_device_free(tb);
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

LinearPart linear_part_from_pack(const std::unordered_map<std::string, Tensor>& pack,
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
  LinearPart p;
  p.w = w.ptr<int8_t>();
  p.scale = sc.ptr<float>();
  p.bias = b.ptr<float>();
  p.out = out;
  p.in = in;
  return p;
}

QLinear qlinear_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                          const std::string& base, int64_t in, int64_t out) {
  return QLinear(std::vector<LinearPart>{linear_part_from_pack(pack, base, in, out)});
}

DeviceFloats::DeviceFloats(size_t n) {
  void* p = nullptr;
  check(sdq_device_alloc(n * sizeof(float), &p), "DeviceFloats");
  p_ = static_cast<float*>(p);
}

DeviceFloats& DeviceFloats::operator=(DeviceFloats&& o) noexcept {
  if (this != &o) {
    sdq_device_free(p_);
    p_ = o.p_;
    o.p_ = nullptr;
  }
  return *this;
}

DeviceFloats::~DeviceFloats() { sdq_device_free(p_); }

namespace {

// A pack entry's values as floats (to_f32 for BF16, src/core/tensor.cpp:44-53).
std::vector<float> entry_floats(const Tensor& t) {
  const int64_t n = t.numel();
  std::vector<float> v((size_t)n);
  if (t.dtype == DType::F32) {
    std::memcpy(v.data(), t.data, (size_t)n * sizeof(float));
  } else {
    const uint16_t* h = static_cast<const uint16_t*>(t.data);
    for (int64_t i = 0; i < n; i++) {
      const uint32_t bits = (uint32_t)h[i] << 16;
      std::memcpy(&v[(size_t)i], &bits, 4);
    }
  }
  return v;
}

}  // namespace

Linear::Linear(const float* w_out_in, const float* bias, int64_t out, int64_t in)
    : in_(in), out_(out), f32_(true) {
  if (!w_out_in || out <= 0 || in < 0) throw std::runtime_error("Linear: bad fp32 weight");
  std::vector<float> t((size_t)(in * out));
  for (int64_t o = 0; o < out; o++)
    for (int64_t i = 0; i < in; i++) t[(size_t)(i * out + o)] = w_out_in[o * in + i];
  if (!t.empty()) {
    w_ = DeviceFloats(t.size());
    check(sdq_memcpy(w_.get(), t.data(), t.size() * sizeof(float), SDQ_H2D, nullptr),
          "Linear weight upload");
  }
  if (bias) {
    b_ = DeviceFloats((size_t)out);
    check(sdq_memcpy(b_.get(), bias, (size_t)out * sizeof(float), SDQ_H2D, nullptr),
          "Linear bias upload");
  }
  check(sdq_stream_sync(nullptr), "Linear upload");
}

Linear::Linear(QLinear&& q) : q_(std::move(q)) {
  in_ = q_.in_features();
  out_ = q_.out_features();
}

void Linear::forward_device(const float* x, int64_t M, float* y, void* stream) const {
  if (!f32_) {
    q_.forward_device(x, M, SDQ_EPI_NONE, nullptr, nullptr, y, stream);
    return;
  }
  check(sdq_linear_f32(x, M, in_, w_.get(), out_, b_.get(), y, stream), "Linear::forward_device");
}

void Linear::mlin(const Tensor& x, Tensor& y) const {
  if (!f32_) {
    q_.mlin(x, y);
    return;
  }
  if (x.dtype != DType::F32) throw std::runtime_error("Linear: x must be F32");
  const int64_t M = x.rows(), K = x.cols();
  if (K != in_)
    throw std::runtime_error("Linear: x has " + std::to_string(K) + " columns, weight expects " +
                             std::to_string(in_));
  y = Tensor({M, out_}, DType::F32);
  if (M == 0) return;
  DeviceFloats dx((size_t)std::max<int64_t>(M * K, 1)), dy((size_t)(M * out_));
  if (M * K > 0)
    check(sdq_memcpy(dx.get(), x.data, (size_t)(M * K) * sizeof(float), SDQ_H2D, nullptr),
          "Linear x");
  forward_device(dx.get(), M, dy.get(), nullptr);
  check(sdq_memcpy(y.data, dy.get(), (size_t)(M * out_) * sizeof(float), SDQ_D2H, nullptr),
        "Linear y");
  check(sdq_stream_sync(nullptr), "Linear");
}

Linear linear_from_pack(const std::unordered_map<std::string, Tensor>& pack,
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
  if (w.dtype == DType::I8) return Linear(qlinear_from_pack(pack, base, in, out));
  const std::vector<float> wf = entry_floats(w);
  const Tensor& b = get(base + ".bias");
  if (b.shape.size() != 1 || b.shape[0] != out || b.dtype == DType::I8)
    throw std::runtime_error("ovi_dit: bad shape for " + base + ".bias");
  const std::vector<float> bf = entry_floats(b);
  return Linear(wf.data(), bf.data(), out, in);
}

}  // namespace gpu
}  // namespace sd
