// CPU ORACLE — test infrastructure only (never linked by the shipped library).
//
// C wrapper around the REFERENCE's own sources, compiled in place from
// /root/reference by oracle/Makefile into oracle/_ref/libsdref.so:
//   src/core/qgemm.cpp   (sd::qgemm, the hot path)
//   src/core/tensor.cpp  (Tensor, parallel_for, quantize_rowwise, randu)
//   src/serde/sdcpp.cpp  (load_sdcpp, the .sdcpp v1 reader)
// Only this wrapper is ours; it builds non-owning sd::Tensor views over the
// caller's buffers so the reference code runs unmodified on them.
#include "core/tensor.h"
#include "serde/sdcpp.h"

#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <string>

namespace {

sd::Tensor view(const void* p, std::initializer_list<int64_t> shape, sd::DType dt, size_t esz) {
  sd::Tensor t;
  t.shape = shape;
  t.dtype = dt;
  t.data = const_cast<void*>(p);
  int64_t n = 1;
  for (auto d : shape) n *= d;
  t.nbytes = (size_t)n * esz;
  t.owning = false;
  return t;
}

}  // namespace

extern "C" {

void sdref_set_nthreads(int n) { sd::set_nthreads(n); }
int sdref_nthreads(void) { return sd::nthreads(); }

// sd::qgemm (src/core/qgemm.cpp:73) on caller buffers; out is [M,N] f32.
int sdref_qgemm(const float* A, const int8_t* Bq, const float* bs, int64_t M, int64_t K,
                int64_t N, float* out) {
  try {
    sd::Tensor a = view(A, {M, K}, sd::DType::F32, 4);
    sd::Tensor b = view(Bq, {N, K}, sd::DType::I8, 1);
    sd::Tensor s = view(bs, {N}, sd::DType::F32, 4);
    sd::Tensor o;
    sd::qgemm(a, b, s, o);
    std::memcpy(out, o.data, (size_t)(M * N) * 4);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// sd::matmul (src/core/gemm.cpp:115): C[M,N] = A[M,K] . B[K,N] (+ bias[N]),
// the fp32 Linear of blk::linear (src/model/blocks.cpp:14-16).
int sdref_matmul(const float* A, int64_t M, int64_t K, const float* B, int64_t N,
                 const float* bias, float* out) {
  try {
    sd::Tensor a = view(A, {M, K}, sd::DType::F32, 4);
    sd::Tensor b = view(B, {K, N}, sd::DType::F32, 4);
    sd::Tensor o;
    sd::matmul(a, b, o, bias);
    if (M * N > 0) std::memcpy(out, o.data, (size_t)(M * N) * 4);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// sd::quantize_rowwise (src/core/tensor.cpp:63).
int sdref_quantize_rowwise(const float* W, int64_t N, int64_t K, int8_t* q, float* s) {
  sd::Tensor w = view(W, {N, K}, sd::DType::F32, 4);
  sd::Tensor wq, sc;
  sd::quantize_rowwise(w, wq, sc);
  std::memcpy(q, wq.data, (size_t)(N * K));
  std::memcpy(s, sc.data, (size_t)N * 4);
  return 0;
}

// sd::randu (src/core/tensor.cpp:125).
void sdref_randu(float* x, int64_t n, uint64_t seed) {
  sd::Tensor t = view(x, {n}, sd::DType::F32, 4);
  sd::randu(t, seed);
}

// sd::load_sdcpp (src/serde/sdcpp.cpp:47). Looks up `name` and reports its
// dtype (0 = I8, 2 = ... as sd::DType), dims and the byte offset of its data
// (and of "<name>.scale" for I8 entries) from the start of the file.
// Returns 0 on success, 1 if the name is absent, -1 if the loader throws
// (message copied into err).
int sdref_sdcpp_lookup(const char* path, const char* name, int* dtype, int64_t* dims,
                       int* ndim, int64_t* data_off, int64_t* scale_off, int* count,
                       char* err, int errlen) {
  try {
    std::shared_ptr<void> owner;
    auto m = sd::load_sdcpp(path, owner);
    *count = (int)m.size();
    auto it = m.find(name);
    if (it == m.end()) return 1;
    const sd::Tensor& t = it->second;
    *dtype = (int)t.dtype;
    *ndim = (int)t.shape.size();
    for (size_t i = 0; i < t.shape.size() && i < 8; i++) dims[i] = t.shape[i];
    const char* base = (const char*)owner.get();
    *data_off = (int64_t)((const char*)t.data - base);
    *scale_off = -1;
    auto is = m.find(std::string(name) + ".scale");
    if (is != m.end()) *scale_off = (int64_t)((const char*)is->second.data - base);
    return 0;
  } catch (const std::exception& e) {
    if (err && errlen > 0) {
      std::strncpy(err, e.what(), (size_t)errlen - 1);
      err[errlen - 1] = 0;
    }
    return -1;
  }
}

}  // extern "C"
