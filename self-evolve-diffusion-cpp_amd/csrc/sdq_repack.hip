// One-time weight repack: .sdcpp int8 [N,K] row-major + f32 [N] scales ->
// MFMA fragment layout (see sdq_internal.h) + zero-padded aligned scales.
//
// The source is the I8 blob of a .sdcpp v1 entry (src/serde/sdcpp.cpp:1-8,
// 107-131; written by tools/quantize/pack_sdcpp.py:90-124): torch Linear
// [out, in] kept as-is, exactly what sd::qgemm consumes as Bq [N, K]
// (src/model/ovi_dit.cpp:40-50, 397-415). One wave writes one 1 KB fragment.
#include "sdq_internal.h"

namespace sdq {
namespace {

__global__ void __launch_bounds__(256)
repack_kernel(const int8_t* __restrict__ q, int64_t N, int64_t K, int64_t KFp, int64_t nfrags,
              int vec, int8_t* __restrict__ frags) {
  const int64_t f = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (f >= nfrags) return;
  const int l = threadIdx.x & 63;
  const int64_t rb = f / KFp, kb = f - rb * KFp;
  const int64_t row = rb * 32 + (l & 31);
  const int64_t k0 = kb * 32 + (l >> 5) * 16;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row < N) {
    const int8_t* src = q + row * K;
    if (vec && k0 + 16 <= K) {
      v = *reinterpret_cast<const uint4*>(src + k0);
    } else {
      uint32_t w[4] = {0, 0, 0, 0};
      for (int e = 0; e < 16; e++)
        if (k0 + e < K) w[e >> 2] |= (uint32_t)(uint8_t)src[k0 + e] << (8 * (e & 3));
      v = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  *reinterpret_cast<uint4*>(frags + f * 1024 + l * 16) = v;
}

__global__ void __launch_bounds__(256)
unpack_kernel(const int8_t* __restrict__ frags, int64_t N, int64_t K, int64_t KFp, int64_t nfrags,
              int8_t* __restrict__ q) {
  const int64_t f = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (f >= nfrags) return;
  const int l = threadIdx.x & 63;
  const int64_t rb = f / KFp, kb = f - rb * KFp;
  const int64_t row = rb * 32 + (l & 31);
  const int64_t k0 = kb * 32 + (l >> 5) * 16;
  if (row >= N) return;
  const uint4 v = *reinterpret_cast<const uint4*>(frags + f * 1024 + l * 16);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  for (int e = 0; e < 16; e++)
    if (k0 + e < K) q[row * K + k0 + e] = (int8_t)(w[e >> 2] >> (8 * (e & 3)));
}

// scale_out[i] = scale[i] for i < N, 0 for N <= i < Np. `scale` may have any
// byte alignment (a .sdcpp blob has no padding), so it is read bytewise.
__global__ void __launch_bounds__(256)
scale_pad_kernel(const uint8_t* __restrict__ scale, int64_t N, int64_t Np,
                 float* __restrict__ scale_out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= Np) return;
  uint32_t u = 0;
  if (i < N) {
    const uint8_t* p = scale + i * 4;
    u = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
  }
  scale_out[i] = __uint_as_float(u);
}

}  // namespace

hipError_t launch_repack_weight(const int8_t* q, const float* scale, int64_t N, int64_t K,
                                int64_t Np, int64_t KFp, int8_t* frags, float* scale_out,
                                hipStream_t s) {
  const int64_t nfrags = (Np / kFragRows) * KFp;
  const int vec = ((reinterpret_cast<uintptr_t>(q) & 15) == 0 && (K % 16) == 0) ? 1 : 0;
  hipLaunchKernelGGL(repack_kernel, dim3((unsigned)ceil_div(nfrags, 4)), dim3(256), 0, s, q, N, K,
                     KFp, nfrags, vec, frags);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(scale_pad_kernel, dim3((unsigned)ceil_div(Np, 256)), dim3(256), 0, s,
                     reinterpret_cast<const uint8_t*>(scale), N, Np, scale_out);
  return hipGetLastError();
}

hipError_t launch_unpack_weight(const int8_t* frags, int64_t N, int64_t K, int64_t KFp, int8_t* q,
                                hipStream_t s) {
  const int64_t nfrags = ceil_div(N, kFragRows) * KFp;
  if (nfrags == 0) return hipSuccess;
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)ceil_div(nfrags, 4)), dim3(256), 0, s, frags, N,
                     K, KFp, nfrags, q);
  return hipGetLastError();
}

}  // namespace sdq
