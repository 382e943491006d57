// sd::Tensor's out-of-line members (host mirror of the reference's
// src/core/tensor.cpp:17-37). sd::qgemm lives in qgemm.cpp, so that a build
// of the reference can link its own tensor.cpp with the GPU qgemm alone.
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>

#include "sd/tensor.h"

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

}  // namespace sd
