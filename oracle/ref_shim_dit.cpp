// CPU ORACLE — test infrastructure only (never linked by the shipped library).
//
// C wrappers around the REFERENCE's DiT glue that sits next to the int8
// Linears: blk::layernorm (src/model/blocks.cpp:18-43) and mod_rows
// (src/model/ovi_dit.cpp:161-172). mod_rows has internal linkage, so this
// translation unit compiles the reference's ovi_dit.cpp itself, in place
// (oracle/Makefile passes -I<reference>/src); only the wrappers are ours.
#include "model/ovi_dit.cpp"

namespace {

sd::Tensor fview(const float* p, std::initializer_list<int64_t> shape) {
  sd::Tensor t;
  t.shape = shape;
  t.dtype = sd::DType::F32;
  t.data = const_cast<float*>(p);
  int64_t n = 1;
  for (auto d : shape) n *= d;
  t.nbytes = (size_t)n * 4;
  t.owning = false;
  return t;
}

}  // namespace

extern "C" {

// blk::layernorm(x, y, nullptr, nullptr, eps) on caller buffers [M,N].
int sdref_layernorm(const float* x, int64_t M, int64_t N, float eps, float* y) {
  try {
    sd::Tensor out;
    sd::blk::layernorm(fview(x, {M, N}), out, nullptr, nullptr, eps);
    std::memcpy(y, out.data, (size_t)(M * N) * 4);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// mod_rows(x, shift, scale, y): y = x*(1+scale)+shift, [L,C] with [C] rows.
int sdref_mod_rows(const float* x, const float* shift, const float* scale, int64_t L, int64_t C,
                   float* y) {
  try {
    sd::Tensor out;
    sd::ovi::mod_rows(fview(x, {L, C}), fview(shift, {C}), fview(scale, {C}), out);
    std::memcpy(y, out.data, (size_t)(L * C) * 4);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

}  // extern "C"
