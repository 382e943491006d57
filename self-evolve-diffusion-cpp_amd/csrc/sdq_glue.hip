// DiT block glue next to the int8 Linears (gfx950): the q / k rmsnorm and
// rotary embedding of the self-attention (src/model/ovi_dit.cpp:182-185,
// src/core/tensor.cpp:112-123 rmsnorm, src/model/blocks.cpp:86-100
// apply_rope), bit-exact with the reference build:
//   ss  = serial float sum of fl(v*v) over the row (not contracted)
//   inv = 1/sqrtf(ss/C + eps);  y = fl(fl(v*inv) * w[c])
//   each head's pair j < nr: (y0, y1) -> (fmaf(y0, c, -fl(y1*s)),
//                                         fmaf(y0, s, fl(y1*c)))
// with c, s = cosf / sinf of the pair's angle, given as a table computed by
// the host with the reference's own libm calls (apply_rope evaluates
// std::cos / std::sin of float angles).
#include "sdq_internal.h"
#include "sdq_rowsum.h"

#pragma clang fp contract(off)

namespace sdq {
namespace {

using rowsum::kLnDepthFew;
using rowsum::kLnDepthMany;
using rowsum::ln_pass;

// inv[row] = 1/sqrtf(sum_k fl(x[row,k]^2)/C + eps), rows of stride ld.
template <bool VEC, int D>
__global__ void __launch_bounds__(64)
rms_stats_kernel(const float* __restrict__ x, int64_t L, int64_t C, int64_t ld, float eps,
                 float* __restrict__ inv) {
  __shared__ float4 tb[2][64];
  const int l = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * 8 + (l & 7);
  const bool ok = row < L;
  const float* r = x + (ok ? row : 0) * ld;
  const float ss = ln_pass<VEC, 2, D>(r, C, l, tb, 0.f);
  if (l < 8 && ok) {
    const float den = ss / (float)C + eps;
    inv[row] = 1.f / sqrtf(den);
  }
}

// y = fl(fl(v*inv)*w) over the row, then the rotation of each head's first
// nr pairs. One thread per pair; pairs never straddle heads (hd is even).
__global__ void __launch_bounds__(256)
rms_rope_apply_kernel(float* __restrict__ x, int64_t L, int64_t C, int64_t ld,
                      const float* __restrict__ w, const float* __restrict__ inv,
                      const float2* __restrict__ cs, int nr, int hd) {
  const int64_t np = C / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= L * np) return;
  const int64_t row = idx / np, p = idx - row * np;
  const int64_t c0 = 2 * p;
  float* q = x + row * ld + c0;
  const float iv = inv[row];
  const float a = q[0] * iv, b = q[1] * iv;
  float y0 = a * w[c0], y1 = b * w[c0 + 1];
  const int j = (int)(c0 % hd) / 2;  // pair index inside the head
  if (cs && j < nr) {
    const float2 t = cs[row * nr + j];  // (cos, sin)
    const float r1s = y1 * t.y, r1c = y1 * t.x;
    const float n0 = __builtin_fmaf(y0, t.x, -r1s);
    const float n1 = __builtin_fmaf(y0, t.y, r1c);
    y0 = n0;
    y1 = n1;
  }
  q[0] = y0;
  q[1] = y1;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

hipError_t launch_rmsnorm_rope(float* x, int64_t L, int64_t C, int64_t ld, const float* w,
                               float eps, int heads, const float* cs, int nr, float* inv,
                               hipStream_t s) {
  if (L <= 0) return hipSuccess;
  if (C <= 0 || ld < C || heads <= 0 || C % heads || (C / heads) % 2 || nr < 0 ||
      nr > C / heads / 2 || !w || !inv)
    return hipErrorInvalidValue;
  const bool vec = aligned16(x) && ld % 4 == 0 && C % 4 == 0, few = L <= 4096;
  const dim3 g((unsigned)ceil_div(L, 8)), b(64);
  if (vec && few)
    hipLaunchKernelGGL((rms_stats_kernel<true, kLnDepthFew>), g, b, 0, s, x, L, C, ld, eps, inv);
  else if (vec)
    hipLaunchKernelGGL((rms_stats_kernel<true, kLnDepthMany>), g, b, 0, s, x, L, C, ld, eps, inv);
  else if (few)
    hipLaunchKernelGGL((rms_stats_kernel<false, kLnDepthFew>), g, b, 0, s, x, L, C, ld, eps, inv);
  else
    hipLaunchKernelGGL((rms_stats_kernel<false, kLnDepthMany>), g, b, 0, s, x, L, C, ld, eps, inv);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t items = L * (C / 2);
  hipLaunchKernelGGL(rms_rope_apply_kernel, dim3((unsigned)ceil_div(items, 256)), dim3(256), 0, s,
                     x, L, C, ld, w, inv, reinterpret_cast<const float2*>(cs), nr,
                     (int)(C / heads));
  return hipGetLastError();
}

}  // namespace sdq
