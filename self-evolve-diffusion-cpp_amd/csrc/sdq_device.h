// Device-side helpers shared by the GEMM translation units (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sdq {

// Per-column operands of the persistent kernel, read by LDS-DMA.
struct ColOps {
  const float* scale;  // [>= tiles_n*BN + 256] zero padded
  const float* bias;   // same size, or nullptr
  const float* gate;   // same size, or nullptr
};

namespace dev {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] |
// vmcnt[5:4] at [15:14]; the other counters are left at their maximum).
constexpr int waitcnt_vm(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (15 << 8); }

// One activation value -> int8 (src/core/qgemm.cpp:62-69, 94): y = v*inv,
// round half to even; NaN and |t| >= 2^31 give -127 (x86 cvtss2si returns
// INT_MIN, which the clamp maps to -127); else clamp to [-127, 127].
__device__ __forceinline__ int quant_one(float v, float inv) {
  const float y = v * inv;
  const float t = __builtin_rintf(y);  // v_rndne_f32: ties to even
  // NaN and |t| >= 2^31 fail this test, like cvtss2si returning INT_MIN.
  if (!(t >= -2147483648.0f && t < 2147483648.0f)) return -127;
  const float c = t < -127.f ? -127.f : (t > 127.f ? 127.f : t);
  return (int)c;
}

__device__ __forceinline__ float gelu_tanh(float v) {
  // nn.GELU(approximate='tanh'), src/model/ovi_dit.cpp:132-142:
  //   0.5 v (1 + tanh(u)) = v / (1 + e^(-2u)),  u = sqrt(2/pi) (v + 0.044715 v^3)
  // (1 + tanh(u) = 2 / (1 + e^(-2u))), with the hardware exp2 and reciprocal
  // (~1 ulp each): a few instructions and no branch. Saturation matches the
  // tanh form: e^(-2u) -> inf gives v * 0 (a signed zero), -> 0 gives v.
  const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  const float e = __builtin_amdgcn_exp2f(-2.8853900817779268f * u);  // e^(-2u) = 2^(-2u log2 e)
  return v * __builtin_amdgcn_rcpf(1.f + e);
}

// Raw buffer descriptor as an SGPR quad (base, range, 32-bit format) and
// the 16-byte-per-lane LDS-DMA load, written as inline asm so that the
// compiler does not track it: it would otherwise assume every LDS read may
// alias every LDS-DMA in flight and drain vmcnt before each read. The
// kernel orders these loads itself (explicit vmcnt waits + barriers).
typedef unsigned v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4u raw_rsrc(const void* base, uint32_t range) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  v4u r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)p);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32) & 0xffffu);
  r.z = __builtin_amdgcn_readfirstlane(range);
  r.w = 0x00020000u;  // gfx9 raw buffer: 32-bit data format
  return r;
}
// The compiler does not see hazards on inline-asm operands: an M0 write
// needs 1 wait state before an LDS-DMA, and a VALU write of an SGPR
// (v_readfirstlane, or v_readlane reloading a spilled SGPR) 5 before a
// vector-memory instruction reads that SGPR. NOP is the asm's leading
// s_nop count: 0 covers M0 and is 4-5% faster in the main loop; 4 covers
// both, for kernels whose SGPR spill reloads can land next to a DMA. The
// CPU test suite scans every compiled kernel for both hazards.
template <int NOP>
__device__ __forceinline__ void dma16(v4u rsrc, uint32_t voff, uint32_t soff, uint32_t lds_addr) {
  static_assert(NOP == 0 || NOP == 4, "s_nop count");
  if constexpr (NOP == 0)
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_addr));
  else
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_addr));
}
__device__ __forceinline__ uint32_t lds_addr32(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(p);
}

}  // namespace dev
}  // namespace sdq
