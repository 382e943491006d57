// fp32 Linear on the GPU: the F32 branch of the reference's `mlin`
// (src/model/ovi_dit.cpp:66-84 -> blk::linear, src/model/blocks.cpp:14-16 ->
// sd::matmul, src/core/gemm.cpp:115-160), for the Linears whose weights a
// pack keeps in fp32 (fewer than 65536 values, e.g. the audio head
// [20, 3072]).
//
// y[i, j] = fl(c + b[j]) with c the serial chain
//   c = +0;  c = fmaf(x[i, k], w[k, j], c)  for k = 0 .. K-1 in order
// which is what the reference's register-tiled matmul computes per output
// (row_group, gemm.cpp:45-75: one fused multiply-add per k into an
// accumulator cleared to +0, then the separate add_bias pass, gemm.cpp:33-40).
// The same chain is also what its scalar loop gives on an FMA target. The
// OpenBLAS path the reference takes above 64M multiply-adds when built with
// OpenBLAS sums in its own order and is not reproduced.
//
// The chain is serial, so a call is latency-bound: each lane owns R outputs
// of one column (R independent chains), the 64 lanes of a wave 64
// consecutive columns (coalesced weight rows), and the loop moves 8 k-steps
// of loads ahead of their multiply-adds.
#include "sdq_internal.h"

#pragma clang fp contract(off)

namespace sdq {
namespace {

constexpr int kUnroll = 8;

template <int R>
__global__ void __launch_bounds__(256)
linear_f32_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                  const float* __restrict__ w, int64_t N, const float* __restrict__ bias,
                  float* __restrict__ y) {
  const int64_t j = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
  const int64_t i0 = ((int64_t)blockIdx.y * 4 + (threadIdx.x >> 6)) * R;
  if (i0 >= M) return;  // uniform per wave
  const bool jok = j < N;
  const int64_t jc = jok ? j : N - 1;  // masked lanes read a valid column
  const float* xr[R];
#pragma unroll
  for (int r = 0; r < R; r++) xr[r] = x + (i0 + r < M ? i0 + r : M - 1) * K;
  const float* wc = w + jc;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.f;
  int64_t k = 0;
  for (; k + kUnroll <= K; k += kUnroll) {
    float wv[kUnroll], xv[R][kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) wv[u] = wc[(k + u) * N];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int u = 0; u < kUnroll; u++) xv[r][u] = xr[r][k + u];
#pragma unroll
    for (int u = 0; u < kUnroll; u++)
#pragma unroll
      for (int r = 0; r < R; r++) acc[r] = __builtin_fmaf(xv[r][u], wv[u], acc[r]);
  }
  for (; k < K; k++) {
    const float wk = wc[k * N];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = __builtin_fmaf(xr[r][k], wk, acc[r]);
  }
  if (!jok) return;
  const float b = bias ? bias[j] : 0.f;
#pragma unroll
  for (int r = 0; r < R; r++) {
    if (i0 + r >= M) break;
    float v = acc[r];
    if (bias) v = v + b;
    y[(i0 + r) * N + j] = v;
  }
}

}  // namespace

hipError_t launch_linear_f32(const float* x, int64_t M, int64_t K, const float* w, int64_t N,
                             const float* bias, float* y, int cu_count, hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  const int64_t col_blocks = ceil_div(N, 64);
  // One output per lane while that still leaves the chip's SIMDs (4 per CU)
  // a few waves each; more rows per lane (independent chains) beyond.
  const int64_t simds = 4 * (cu_count > 0 ? cu_count : 256);
  const bool one = col_blocks * M <= 4 * simds;
  const int R = one ? 1 : 4;
  const int64_t row_blocks = ceil_div(M, 4 * R);
  if (row_blocks > 65535 || col_blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid((unsigned)col_blocks, (unsigned)row_blocks);
  if (one)
    hipLaunchKernelGGL(linear_f32_kernel<1>, grid, dim3(256), 0, s, x, M, K, w, N, bias, y);
  else
    hipLaunchKernelGGL(linear_f32_kernel<4>, grid, dim3(256), 0, s, x, M, K, w, N, bias, y);
  return hipGetLastError();
}

}  // namespace sdq
