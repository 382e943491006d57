// A caller written against the reference's own core header
// (src/core/tensor.h), built from the reference's src/core/tensor.cpp and
// linked with libsd_qgemm.so in place of src/core/qgemm.cpp: the drop-in as a
// reference maintainer would wire it (the Makefile's SRCS minus qgemm.cpp).
// Every sd::Tensor member comes from the reference's tensor.cpp; sd::qgemm
// runs on the GPU.
//
// usage: ref_caller M K N seedA seedW out.bin
// Fills A [M,K] and W [N,K] with the reference's randu, quantizes W with its
// quantize_rowwise, calls sd::qgemm, and writes M, K, N (int64) then A (f32),
// Wq (i8), scales (f32) and the output (f32) to out.bin for the test to check
// against the reference's own qgemm.
#include <cstdio>
#include <cstdlib>

#include "core/tensor.h"
#include "sdq.h"

static bool put(std::FILE* f, const void* p, size_t n) { return std::fwrite(p, 1, n, f) == n; }

int main(int argc, char** argv) {
  if (argc != 7) {
    std::fprintf(stderr, "usage: %s M K N seedA seedW out.bin\n", argv[0]);
    return 2;
  }
  const int64_t M = std::atoll(argv[1]), K = std::atoll(argv[2]), N = std::atoll(argv[3]);
  const uint64_t seed_a = std::strtoull(argv[4], nullptr, 10);
  const uint64_t seed_w = std::strtoull(argv[5], nullptr, 10);
  if (sdq_init(0) != SDQ_OK) {
    std::fprintf(stderr, "sdq_init: %s\n", sdq_last_error());
    return 1;
  }
  sd::Tensor A({M, K}, sd::DType::F32), W({N, K}, sd::DType::F32);
  sd::randu(A, seed_a);
  sd::randu(W, seed_w);
  sd::Tensor Wq, sc;
  sd::quantize_rowwise(W, Wq, sc);
  sd::Tensor out;
  try {
    sd::qgemm(A, Wq, sc, out);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "qgemm: %s\n", e.what());
    return 1;
  }
  if (out.rows() != M || out.cols() != N || out.dtype != sd::DType::F32) {
    std::fprintf(stderr, "qgemm: bad output shape\n");
    return 1;
  }
  std::FILE* f = std::fopen(argv[6], "wb");
  if (!f) return 1;
  const int64_t dims[3] = {M, K, N};
  const bool ok = put(f, dims, sizeof dims) && put(f, A.data, A.nbytes) &&
                  put(f, Wq.data, Wq.nbytes) && put(f, sc.data, sc.nbytes) &&
                  put(f, out.data, out.nbytes);
  std::fclose(f);
  std::printf("ref_caller: qgemm M=%lld K=%lld N=%lld done\n", (long long)M, (long long)K,
              (long long)N);
  return ok ? 0 : 1;
}
