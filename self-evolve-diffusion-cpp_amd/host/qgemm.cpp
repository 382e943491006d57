// sd::qgemm on the GPU: the drop-in for the reference's src/core/qgemm.cpp
// (same signature and result, bit for bit; declaration in sd/tensor.h,
// the reference's in src/core/tensor.h:48-52). It uses sd::Tensor through its
// inline members and its constructor, destructor, move assignment and
// numel(), and defines none of them: libsd_qgemm.so is this file alone, so a
// program built from the reference's own src/core/tensor.cpp links it in
// place of qgemm.cpp with one definition of every Tensor member.
#include <cstdint>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>

#include "sd/tensor.h"
#include "sdq.h"

namespace sd {

namespace {

void check_rc(int rc, const char* what) {
  if (rc != SDQ_OK) throw std::runtime_error(std::string(what) + ": " + sdq_last_error());
}

// Device copies of (Bq, bs), keyed by the host views' addresses.
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
  check_rc(sdq_weight_upload(Bq.ptr<int8_t>(), bs.ptr<float>(), N, K, nullptr, &w),
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
  check_rc(sdq_qlinear_host(w, A.ptr<float>(), M, K, nullptr, out.data), "qgemm");
}

}  // namespace sd
