// sd::Tensor and sd::qgemm (host mirror of the reference's src/core, int8
// path only). qgemm forwards to the sdq C ABI; see sd/tensor.h.
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>

#include "sd/qlinear.h"
#include "sd/tensor.h"
#include "sdq.h"

namespace sd {

static size_t dtype_size(DType d) {
  switch (d) {
    case DType::F32: return 4;
    case DType::BF16: return 2;
    case DType::I8: return 1;
  }
  return 4;
}

// Owning tensors are 64-byte aligned and zero-filled (src/core/tensor.cpp:19-24).
Tensor::Tensor(std::vector<int64_t> s, DType d) : shape(std::move(s)), dtype(d) {
  int64_t n = 1;
  for (int64_t x : shape) n *= x;
  nbytes = (size_t)n * dtype_size(dtype);
  const size_t cap = ((nbytes + 63) / 64) * 64;
  data = std::aligned_alloc(64, cap ? cap : 64);
  if (!data) throw std::bad_alloc();
  std::memset(data, 0, nbytes);
}

Tensor::~Tensor() {
  if (owning && data) std::free(data);
}

Tensor::Tensor(Tensor&& o) noexcept { *this = std::move(o); }

Tensor& Tensor::operator=(Tensor&& o) noexcept {
  if (this != &o) {
    if (owning && data) std::free(data);
    shape = std::move(o.shape);
    dtype = o.dtype;
    data = o.data;
    nbytes = o.nbytes;
    owning = o.owning;
    o.data = nullptr;
    o.nbytes = 0;
  }
  return *this;
}

int64_t Tensor::numel() const {
  int64_t n = 1;
  for (int64_t x : shape) n *= x;
  return n;
}

void Tensor::reshape(std::vector<int64_t> s) {
  int64_t n = 1;
  for (int64_t x : s) n *= x;
  if (n != numel()) throw std::runtime_error("reshape: numel mismatch");
  shape = std::move(s);
}

// ---- weight cache for the host-tensor qgemm ------------------------------
namespace {

struct WeightKey {
  const void* q;
  const void* s;
  int64_t N, K;
  bool operator<(const WeightKey& o) const {
    return std::tie(q, s, N, K) < std::tie(o.q, o.s, o.N, o.K);
  }
};

std::mutex g_cache_mu;
std::map<WeightKey, sdq_weight*>& cache() {
  static std::map<WeightKey, sdq_weight*> m;
  return m;
}

sdq_weight* cached_weight(const Tensor& Bq, const Tensor& bs, int64_t N, int64_t K) {
  std::lock_guard<std::mutex> lk(g_cache_mu);
  WeightKey key{Bq.data, bs.data, N, K};
  auto it = cache().find(key);
  if (it != cache().end()) return it->second;
  sdq_weight* w = nullptr;
  gpu::check(sdq_weight_upload(Bq.ptr<int8_t>(), bs.ptr<float>(), N, K, nullptr, &w),
             "qgemm: weight upload");
  cache().emplace(key, w);
  return w;
}

}  // namespace

void qgemm_cache_clear() {
  std::lock_guard<std::mutex> lk(g_cache_mu);
  for (auto& kv : cache()) sdq_weight_free(kv.second);
  cache().clear();
}

size_t qgemm_cache_size() {
  std::lock_guard<std::mutex> lk(g_cache_mu);
  return cache().size();
}

void qgemm(const Tensor& A, const Tensor& Bq, const Tensor& bs, Tensor& out) {
  const int64_t M = A.rows(), K = A.cols(), N = Bq.rows();
  if (A.dtype != DType::F32) throw std::runtime_error("qgemm: A must be F32");
  if (Bq.dtype != DType::I8) throw std::runtime_error("qgemm: Bq must be I8");
  if (bs.dtype != DType::F32) throw std::runtime_error("qgemm: bs must be F32");
  if (Bq.cols() != K)
    throw std::runtime_error("qgemm: K mismatch (A cols " + std::to_string(K) + ", Bq cols " +
                             std::to_string(Bq.cols()) + ")");
  if (bs.numel() != N) throw std::runtime_error("qgemm: bs must have N entries");
  out = Tensor({M, N}, DType::F32);
  if (M == 0 || N == 0 || K == 0) return;  // zero-filled, src/core/qgemm.cpp:74-76
  sdq_weight* w = cached_weight(Bq, bs, N, K);
  gpu::check(sdq_qlinear_host(w, A.ptr<float>(), M, K, nullptr, out.data), "qgemm");
}

}  // namespace sd
