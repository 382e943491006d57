// Host-side mirror of the reference's core tensor contract for the int8
// Linear path (reference: src/core/tensor.h). Same names, field meanings and
// ownership rules, so code written against the reference's sd::Tensor and
// sd::qgemm compiles against this header unchanged; sd::qgemm here runs on
// the MI355X through the sdq C ABI (include/sdq.h).
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace sd {

// src/core/tensor.h:13
enum class DType : uint8_t { F32 = 0, BF16 = 1, I8 = 2 };

// Row-major CPU tensor, owning (64-byte aligned, zero-filled) or a
// non-owning view; move-only. src/core/tensor.h:16-38, tensor.cpp:19-37.
struct Tensor {
  std::vector<int64_t> shape;
  DType dtype = DType::F32;
  void* data = nullptr;
  size_t nbytes = 0;
  bool owning = true;

  Tensor() = default;
  Tensor(std::vector<int64_t> s, DType d);
  Tensor(const Tensor&) = delete;
  Tensor& operator=(const Tensor&) = delete;
  Tensor(Tensor&& o) noexcept;
  Tensor& operator=(Tensor&& o) noexcept;
  ~Tensor();

  int64_t numel() const;
  int64_t rows() const { return shape.size() >= 2 ? shape[shape.size() - 2] : 1; }
  int64_t cols() const { return shape.size() >= 1 ? shape[shape.size() - 1] : 1; }
  size_t dim(int i) const { return (size_t)shape[i]; }
  void reshape(std::vector<int64_t> s);
  template <typename T> T* ptr() { return reinterpret_cast<T*>(data); }
  template <typename T> const T* ptr() const { return reinterpret_cast<const T*>(data); }
};

// int8 weight-stationary qGEMM, src/core/tensor.h:48-52:
//   A: F32 [M,K]; Bq: I8 [N,K]; bs: F32 [N]; out := new F32 [M,N].
//   out[i,j] = (float)(sum_k aq[i,k]*Bq[j,k]) * (as[i]*bs[j]) with the
//   reference's per-row dynamic activation quantization — bit-identical.
// Runs on the current HIP device (sdq_init). The device copy of (Bq, bs) is
// uploaded and repacked once and cached by (Bq.data, bs.data, N, K) plus a
// fingerprint of the contents (all of bs, the first and last rows of Bq),
// checked on every call: new contents at a cached address are uploaded
// again. A change confined to Bq's middle rows is not seen, so a caller that
// rewrites weights in place or releases a pack calls qgemm_cache_clear(),
// which also frees the device copies. Safe to call from several threads: a
// device copy that one thread replaces or clears while another thread's call
// uses it is freed when that call returns.
// Unlike the reference, shape mismatches throw std::runtime_error("qgemm: …")
// instead of reading out of bounds; GPU failures throw too.
void qgemm(const Tensor& A, const Tensor& Bq, const Tensor& bs, Tensor& out);
void qgemm_cache_clear();
size_t qgemm_cache_size();

}  // namespace sd
