// sd::qgemm on the GPU: the drop-in for the reference's src/core/qgemm.cpp
// (same signature and result, bit for bit; declaration in sd/tensor.h,
// the reference's in src/core/tensor.h:48-52). It uses sd::Tensor through its
// inline members and its constructor, destructor, move assignment and
// numel(), and defines none of them: libsd_qgemm.so is this file alone, so a
// program built from the reference's own src/core/tensor.cpp links it in
// place of qgemm.cpp with one definition of every Tensor member.
#include <cstdint>
#include <map>
#include <memory>
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

// Device copies of (Bq, bs), keyed by the host views' addresses. A view's
// address can be reused for other contents (a pack unmapped and another
// mapped in its place, weights rewritten in place), so each entry also keeps
// a fingerprint of the contents: all of bs and the first and last rows of
// Bq. A changed fingerprint replaces the device copy. Entries are shared: a
// call holds its weight until it returns, so a copy replaced or cleared by
// another thread meanwhile is freed only after its last user is done.
struct WeightKey {
  const void* q;
  const void* s;
  int64_t N, K;
  bool operator<(const WeightKey& o) const {
    return std::tie(q, s, N, K) < std::tie(o.q, o.s, o.N, o.K);
  }
};
using WeightRef = std::shared_ptr<sdq_weight>;
struct CachedWeight {
  WeightRef w;
  uint64_t print;
};

uint64_t fnv1a(uint64_t h, const void* p, size_t n) {
  const unsigned char* b = static_cast<const unsigned char*>(p);
  for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 0x100000001b3ull;
  return h;
}

uint64_t fingerprint(const Tensor& Bq, const Tensor& bs, int64_t N, int64_t K) {
  uint64_t h = 0xcbf29ce484222325ull;
  h = fnv1a(h, bs.data, (size_t)N * sizeof(float));
  const int8_t* q = Bq.ptr<int8_t>();
  h = fnv1a(h, q, (size_t)K);
  return fnv1a(h, q + (N - 1) * K, (size_t)K);
}

std::mutex g_cache_mu;
// Never destroyed: no device memory is freed while the process exits.
std::map<WeightKey, CachedWeight>& cache() {
  static auto* m = new std::map<WeightKey, CachedWeight>();
  return *m;
}

WeightRef cached_weight(const Tensor& Bq, const Tensor& bs, int64_t N, int64_t K) {
  const uint64_t print = fingerprint(Bq, bs, N, K);
  std::lock_guard<std::mutex> lk(g_cache_mu);
  WeightKey key{Bq.data, bs.data, N, K};
  auto it = cache().find(key);
  if (it != cache().end()) {
    if (it->second.print == print) return it->second.w;
    cache().erase(it);  // freed once no call holds it
  }
  sdq_weight* raw = nullptr;
  check_rc(sdq_weight_upload(Bq.ptr<int8_t>(), bs.ptr<float>(), N, K, nullptr, &raw),
           "qgemm: weight upload");
  WeightRef w(raw, [](sdq_weight* p) { sdq_weight_free(p); });
  cache().emplace(key, CachedWeight{w, print});
  return w;
}

}  // namespace

void qgemm_cache_clear() {
  std::lock_guard<std::mutex> lk(g_cache_mu);
  cache().clear();  // each copy is freed once no call holds it
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
  const WeightRef w = cached_weight(Bq, bs, N, K);  // held until the call has returned
  check_rc(sdq_qlinear_host(w.get(), A.ptr<float>(), M, K, nullptr, out.data), "qgemm");
}

}  // namespace sd
