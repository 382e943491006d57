// Practical ceiling of the int8 MFMA pipe on this GPU (gfx950), for the
// roofline of the qGEMM: v_mfma_i32_32x32x32_i8 or v_mfma_i32_16x16x64_i8
// back to back in every SIMD, one workgroup per CU, operands
//   * random bytes held in registers (no memory traffic), or
//   * random bytes re-read from LDS every k-step with the qGEMM's register
//     double buffering (the operand pattern of its 128n x 64m wave tiles),
//   * zero bytes (the same loop with little switching activity),
// and the LDS read bandwidth of 16-byte reads. Rates come from HIP events
// around the second of two launches (the first warms the clock up). The
// same instruction stream runs on random and on zero operands: the gap
// between the two is the power limit (the clock drops when the operands
// switch), which bounds the GEMM below the 5.0 POPS nominal peak (a
// 32x32x32 i8 MFMA is 65536 ops, 32 cycles per SIMD: 8192 ops/clk/CU; a
// 16x16x64 one is 32768 ops in 16 cycles, the same rate per clock). Two
// forms with the same wave tile and the same LDS bytes per k are compared:
// the 16x16x64 one switches fewer accumulator registers per operation.
// Each kernel also reads s_memtime and s_memrealtime around its loop; their
// ratio is printed as a relative clock reading (higher = faster clock).
//
// Build: make -C self-evolve-diffusion-cpp_amd lib/mfma_ceiling (part of `all`).
// Run:   self-evolve-diffusion-cpp_amd/lib/mfma_ceiling
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <utility>
#include <vector>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));            \
      std::exit(1);                                                           \
    }                                                                         \
  } while (0)

constexpr int kLdsVec = 8192;  // 128 KB of 16-byte words

struct Clocks {
  unsigned long long shader, real;
};

// FN x FM accumulator blocks per wave; READS: the next k-step's FN + FM
// fragments come from LDS while this step's MFMAs run.
template <int FN, int FM, bool READS, int WAVES>
__global__ void __launch_bounds__(WAVES * 64, 1)
mfma_loop(int iters, const int* __restrict__ bytes, int* out, Clocks* clk) {
  __shared__ v4i lds[kLdsVec];
  for (int i = threadIdx.x; i < kLdsVec; i += blockDim.x) {
    const int* r = bytes + ((size_t)blockIdx.x * kLdsVec + i) % (1 << 20) * 4;
    lds[i] = v4i{r[0], r[1], r[2], r[3]};
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v16i acc[FN][FM];
#pragma unroll
  for (int a = 0; a < FN; a++)
#pragma unroll
    for (int b = 0; b < FM; b++) acc[a][b] = v16i{};
  v4i a0[FN], b0[FM], a1[FN], b1[FM];
#pragma unroll
  for (int a = 0; a < FN; a++) a0[a] = a1[a] = lds[(lane + (a + w * 8) * 64) & (kLdsVec - 1)];
#pragma unroll
  for (int b = 0; b < FM; b++) b0[b] = b1[b] = lds[(lane + (b + 4 + w * 8) * 64) & (kLdsVec - 1)];
  const unsigned long long s0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; it++) {
    // two k-steps per iteration, alternating the register sets
#pragma unroll
    for (int i = 0; i < FN * FM; i++) {
      acc[i / FM][i % FM] =
          __builtin_amdgcn_mfma_i32_32x32x32_i8(a0[i / FM], b0[i % FM], acc[i / FM][i % FM], 0, 0, 0);
      if (READS && i < FN)
        a1[i] = lds[(lane + (i + w * 8 + it * 2) * 64) & (kLdsVec - 1)];
      else if (READS && i < FN + FM)
        b1[i - FN] = lds[(lane + (i + w * 8 + it * 2 + 64) * 64) & (kLdsVec - 1)];
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < FN * FM; i++) {
      acc[i / FM][i % FM] =
          __builtin_amdgcn_mfma_i32_32x32x32_i8(a1[i / FM], b1[i % FM], acc[i / FM][i % FM], 0, 0, 0);
      if (READS && i < FN)
        a0[i] = lds[(lane + (i + w * 8 + it * 2 + 1) * 64) & (kLdsVec - 1)];
      else if (READS && i < FN + FM)
        b0[i - FN] = lds[(lane + (i + w * 8 + it * 2 + 65) * 64) & (kLdsVec - 1)];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const unsigned long long s1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  int sum = 0;
#pragma unroll
  for (int a = 0; a < FN; a++)
#pragma unroll
    for (int b = 0; b < FM; b++)
#pragma unroll
      for (int r = 0; r < 16; r++) sum += acc[a][b][r];
  out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
  if (threadIdx.x == 0) clk[blockIdx.x] = Clocks{s1 - s0, r1 - r0};
}

// The same with v_mfma_i32_16x16x64_i8: FN x FM blocks of 16x16 per wave
// (a 32x32 block of the loop above is 2 x 2 of these, so FN x FM here is
// 2FN x 2FM there for the same wave tile).
template <int FN, int FM, bool READS, int WAVES>
__global__ void __launch_bounds__(WAVES * 64, 1)
mfma16_loop(int iters, const int* __restrict__ bytes, int* out, Clocks* clk) {
  __shared__ v4i lds[kLdsVec];
  for (int i = threadIdx.x; i < kLdsVec; i += blockDim.x) {
    const int* r = bytes + ((size_t)blockIdx.x * kLdsVec + i) % (1 << 20) * 4;
    lds[i] = v4i{r[0], r[1], r[2], r[3]};
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v4i acc[FN][FM];
#pragma unroll
  for (int a = 0; a < FN; a++)
#pragma unroll
    for (int b = 0; b < FM; b++) acc[a][b] = v4i{0, 0, 0, 0};
  v4i a0[FN], b0[FM], a1[FN], b1[FM];
#pragma unroll
  for (int a = 0; a < FN; a++) a0[a] = a1[a] = lds[(lane + (a + w * 16) * 64) & (kLdsVec - 1)];
#pragma unroll
  for (int b = 0; b < FM; b++) b0[b] = b1[b] = lds[(lane + (b + 8 + w * 16) * 64) & (kLdsVec - 1)];
  const unsigned long long s0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int i = 0; i < FN * FM; i++) {
      acc[i / FM][i % FM] =
          __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[i / FM], b0[i % FM], acc[i / FM][i % FM], 0, 0, 0);
      if (READS && i < FN)
        a1[i] = lds[(lane + (i + w * 16 + it * 2) * 64) & (kLdsVec - 1)];
      else if (READS && i < FN + FM)
        b1[i - FN] = lds[(lane + (i + w * 16 + it * 2 + 64) * 64) & (kLdsVec - 1)];
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < FN * FM; i++) {
      acc[i / FM][i % FM] =
          __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[i / FM], b1[i % FM], acc[i / FM][i % FM], 0, 0, 0);
      if (READS && i < FN)
        a0[i] = lds[(lane + (i + w * 16 + it * 2 + 1) * 64) & (kLdsVec - 1)];
      else if (READS && i < FN + FM)
        b0[i - FN] = lds[(lane + (i + w * 16 + it * 2 + 65) * 64) & (kLdsVec - 1)];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const unsigned long long s1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  int sum = 0;
#pragma unroll
  for (int a = 0; a < FN; a++)
#pragma unroll
    for (int b = 0; b < FM; b++)
#pragma unroll
      for (int r = 0; r < 4; r++) sum += acc[a][b][r];
  out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
  if (threadIdx.x == 0) clk[blockIdx.x] = Clocks{s1 - s0, r1 - r0};
}

// 16-byte LDS reads, 16 per wave per iteration, conflict free.
template <int WAVES>
__global__ void __launch_bounds__(WAVES * 64, 1)
lds_reads(int iters, int* out, Clocks* clk) {
  __shared__ v4i lds[kLdsVec];
  for (int i = threadIdx.x; i < kLdsVec; i += blockDim.x) lds[i] = v4i{i, 3 * i, 5 * i, 7 * i};
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v4i acc = {0, 0, 0, 0};
  const unsigned long long s0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int j = 0; j < 16; j++) acc ^= lds[(lane + (j * 8 + w) * 64 + it * 64) & (kLdsVec - 1)];
  }
  const unsigned long long s1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  out[blockIdx.x * blockDim.x + threadIdx.x] = acc.x + acc.y + acc.z + acc.w;
  if (threadIdx.x == 0) clk[blockIdx.x] = Clocks{s1 - s0, r1 - r0};
}

int main() {
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  int *out, *rnd, *zero;
  Clocks* clk;
  CHECK(hipMalloc(&out, (size_t)cus * 1024 * sizeof(int)));
  CHECK(hipMalloc(&clk, (size_t)cus * sizeof(Clocks)));
  CHECK(hipMalloc(&rnd, (size_t)(1 << 22) * sizeof(int)));
  CHECK(hipMalloc(&zero, (size_t)(1 << 22) * sizeof(int)));
  std::vector<int> h(1 << 22);
  unsigned x = 12345;
  for (int& v : h) {  // xorshift32: uniformly random bytes
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    v = (int)x;
  }
  CHECK(hipMemcpy(rnd, h.data(), h.size() * sizeof(int), hipMemcpyHostToDevice));
  CHECK(hipMemset(zero, 0, h.size() * sizeof(int)));
  std::vector<Clocks> hc(cus);
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  std::printf("%d CUs\n", cus);
  // Runs `launch` twice (the first warms the clock up), times the second.
  auto timed = [&](auto launch, double per_cu, const char* what, const char* unit) {
    launch();
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(e0));
    launch();
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    CHECK(hipMemcpy(hc.data(), clk, cus * sizeof(Clocks), hipMemcpyDeviceToHost));
    double cyc = 0, real = 0;
    for (const Clocks& c : hc) {
      cyc += (double)c.shader;
      real += (double)c.real;
    }
    cyc /= cus;
    real /= cus;
    std::printf("%-44s %8.3f ms  clock reading %.2f", what, ms, cyc / (real / 100e6) / 1e9);
    (void)unit;
    return std::make_pair(ms, per_cu * cus / (ms * 1e-3));
  };
#define MFMA(FN, FM, READS, WAVES, SRC, NAME)                                                      \
  {                                                                                                \
    const int iters = 4000;                                                                        \
    const double ops = (double)WAVES * iters * 2 * FN * FM * 65536.0;                              \
    auto r = timed(                                                                                \
        [&] {                                                                                      \
          hipLaunchKernelGGL((mfma_loop<FN, FM, READS, WAVES>), dim3(cus), dim3(WAVES * 64), 0, 0, \
                             iters, SRC, out, clk);                                                \
        },                                                                                         \
        ops, NAME, "ops");                                                                         \
    std::printf("  %6.0f TOPS = %.3f of 5.0 POPS\n", r.second / 1e12, r.second / 5.0e15);        \
  }
#define MFMA16(FN, FM, READS, WAVES, SRC, NAME)                                                    \
  {                                                                                                \
    const int iters = 4000;                                                                        \
    const double ops = (double)WAVES * iters * 2 * FN * FM * 32768.0;                              \
    auto r = timed(                                                                                \
        [&] {                                                                                      \
          hipLaunchKernelGGL((mfma16_loop<FN, FM, READS, WAVES>), dim3(cus), dim3(WAVES * 64), 0,  \
                             0, iters, SRC, out, clk);                                             \
        },                                                                                         \
        ops, NAME, "ops");                                                                         \
    std::printf("  %6.0f TOPS = %.3f of 5.0 POPS\n", r.second / 1e12, r.second / 5.0e15);        \
  }
  // the first launch on a cold GPU runs at a lower clock: one untimed pass
  MFMA(4, 2, true, 8, rnd, "(warm-up) 32x32x32, 8 waves, 4x2 blocks")
  MFMA(4, 2, false, 8, rnd, "32x32x32, 8 waves, 4x2 blocks, random, registers")
  MFMA16(8, 4, false, 8, rnd, "16x16x64, 8 waves, 8x4 blocks, random, registers")
  MFMA(4, 2, true, 8, rnd, "32x32x32, 8 waves, 4x2 blocks, random, LDS reads")
  MFMA16(8, 4, true, 8, rnd, "16x16x64, 8 waves, 8x4 blocks, random, LDS reads")
  MFMA(2, 2, true, 8, rnd, "32x32x32, 8 waves, 2x2 blocks, random, LDS reads")
  MFMA16(4, 4, true, 8, rnd, "16x16x64, 8 waves, 4x4 blocks, random, LDS reads")
  MFMA(4, 4, false, 4, rnd, "32x32x32, 4 waves, 4x4 blocks, random, registers")
  MFMA(4, 4, true, 4, rnd, "32x32x32, 4 waves, 4x4 blocks, random, LDS reads")
  MFMA(4, 2, true, 8, zero, "32x32x32, 8 waves, 4x2 blocks, zeros, LDS reads")
  MFMA16(8, 4, true, 8, zero, "16x16x64, 8 waves, 8x4 blocks, zeros, LDS reads")
#define LDS(WAVES)                                                                                 \
  {                                                                                                \
    const int iters = 4000;                                                                        \
    auto r = timed([&] {                                                                           \
      hipLaunchKernelGGL((lds_reads<WAVES>), dim3(cus), dim3(WAVES * 64), 0, 0, iters, out, clk);  \
    }, (double)WAVES * iters * 16 * 1024, "LDS ds_read_b128, " #WAVES " waves", "B");              \
    std::printf("  %6.1f GB/s per CU\n", r.second / cus / 1e9);                                    \
  }
  LDS(4)
  LDS(8)
  LDS(16)
  CHECK(hipFree(out));
  CHECK(hipFree(clk));
  CHECK(hipFree(rnd));
  CHECK(hipFree(zero));
  return 0;
}
