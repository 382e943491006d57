// Serial per-row float sums in column order, the way the reference's CPU
// loops accumulate (bit-exact): the layernorm mean and variance
// (blocks.cpp:18-43) and the rmsnorm sum of squares (tensor.cpp:112-123).
// Device-side helpers shared by the quantizer and the block-glue kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sdq {
namespace rowsum {

// One wave per 8 rows: the 64 lanes load 8-row x 32-column tiles coalesced
// (lane l: row l & 7, 16 bytes at column 4*(l >> 3)), D tiles in flight in
// registers; each tile is transposed through LDS and lanes 0-7 add their
// row's 32 values in order. A row's K dependent adds bound the latency for
// few rows (~700 cycles per 32-column tile); HBM bandwidth for many.
// tiles in flight per wave: 32 for few rows (latency), 16 for many (more
// waves per SIMD; bandwidth-bound there)
constexpr int kLnDepthFew = 32, kLnDepthMany = 16;

// 4 values of row r at columns c .. c+3 (values past K unspecified: see
// mask4); every lane issues its load(s) (the address is clamped into the
// row), so the tile loop has no branches and its loads stay in flight across
// iterations. VEC: K % 4 == 0 and 16-byte aligned rows (one 16-byte load).
template <bool VEC>
__device__ __forceinline__ float4 load4(const float* __restrict__ r, int64_t c, int64_t K) {
  float4 v;
  if constexpr (VEC) {
    v = *reinterpret_cast<const float4*>(r + (c + 4 <= K ? c : K - 4));
  } else {
    v.x = r[c < K ? c : K - 1];
    v.y = r[c + 1 < K ? c + 1 : K - 1];
    v.z = r[c + 2 < K ? c + 2 : K - 1];
    v.w = r[c + 3 < K ? c + 3 : K - 1];
  }
  return v;
}

// Zeroes the values of a load4 result past K. Applied when the tile is
// consumed, not at the load: using the data right away would make every
// prefetched load wait for its own completion.
__device__ __forceinline__ float4 mask4(float4 v, int64_t c, int64_t K) {
  v.x = c < K ? v.x : 0.f;
  v.y = c + 1 < K ? v.y : 0.f;
  v.z = c + 2 < K ? v.z : 0.f;
  v.w = c + 3 < K ? v.w : 0.f;
  return v;
}

// The summed term of value v: v (PASS 0), the rounded (v - mu)^2 (PASS 1),
// the rounded v^2 (PASS 2).
template <int PASS>
__device__ __forceinline__ float ln_term(float v, float mu) {
  if constexpr (PASS == 0) {
    return v;
  } else if constexpr (PASS == 1) {
    const float d = v - mu;
    return d * d;
  } else {
    return v * v;
  }
}

// Serial sum of one 32-column tile of this lane's row (lanes 0-7) from the
// transposed tile of terms in LDS; n = columns of the tile inside the row
// (32 but for the last).
__device__ __forceinline__ float ln_tile_sum(const float4* __restrict__ tb, int l, float acc,
                                             int n) {
  if (n == 32) {
    // all eight reads first (one LDS latency per tile), then the 32 dependent
    // adds back to back
    float4 v[8];
#pragma unroll
    for (int q = 0; q < 8; q++) v[q] = tb[q * 8 + l];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 8; q++) {
      acc = acc + v[q].x;
      acc = acc + v[q].y;
      acc = acc + v[q].z;
      acc = acc + v[q].w;
    }
  } else {
    for (int c = 0; c < n; c++) {
      const float4 v = tb[(c >> 2) * 8 + l];
      const int e = c & 3;
      acc = acc + (e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w)));
    }
  }
  return acc;
}

// For one-wave workgroups only (64 threads: tb is the wave's own tile
// buffer, and no barrier orders other waves). Every lane turns its 4 values
// into terms before the tile goes to LDS (PASS 1 needs the row's mean in
// every lane: lane l holds row l & 7), so the 8 adding lanes run only the
// chain of dependent adds.
template <bool VEC, int PASS, int D>
__device__ __forceinline__ float ln_pass(const float* __restrict__ r, int64_t K, int l,
                                         float4 (&tb)[2][64], float mu) {
  const int j = l >> 3;
  const int64_t nt = (K + 31) / 32;
  float acc = 0.f;
  float4 buf[D];
#pragma unroll
  for (int u = 0; u < D; u++) buf[u] = load4<VEC>(r, (int64_t)u * 32 + 4 * j, K);
  for (int64_t t0 = 0; t0 < nt; t0 += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const int64_t t = t0 + u;
      float4 v = mask4(buf[u], t * 32 + 4 * j, K);
      if constexpr (PASS != 0) {
        // columns past K: never summed (ln_tile_sum adds n terms)
        v.x = ln_term<PASS>(v.x, mu);
        v.y = ln_term<PASS>(v.y, mu);
        v.z = ln_term<PASS>(v.z, mu);
        v.w = ln_term<PASS>(v.w, mu);
      }
      tb[t & 1][l] = v;
      buf[u] = load4<VEC>(r, (t + D) * 32 + 4 * j, K);
      // The workgroup is one wave (64 threads): its LDS operations execute
      // in issue order, so waiting for the tile's LDS write is enough. A
      // __syncthreads() would also wait for every global load in flight,
      // draining the D-deep prefetch at each tile.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (l < 8 && t < nt) {
        const int n = (int)((K - t * 32) < 32 ? (K - t * 32) : 32);
        acc = ln_tile_sum(tb[t & 1], l, acc, n);
      }
    }
  }
  return acc;
}


// Full tiles (K % 32 == 0, 16-byte aligned rows) through a buffer
// descriptor over the rows (range: the bytes the rows span, below 2^31):
// lane l loads at voff (its row's byte offset, or the range itself for a
// row past the end) plus 128 bytes per tile, and loads past the range return
// 0 without touching memory, so the loop needs no address clamps and no
// column masks (tiles past the row end are loaded but never summed). Three
// LDS buffers: iteration t reads tile t+1 (written and waited in iteration
// t-1), writes tile t+2, adds tile t from registers, then waits, so the LDS
// latency runs under the adds. D (a multiple of 6) tiles of loads in
// flight. Same sums, in the same order, as ln_pass; every lane returns the
// sum of its row (l & 7).
typedef float v4f_rs __attribute__((ext_vector_type(4)));
constexpr int kLnDepthFull = 12;
// Largest range: voff + (nt + 2D + 2) * 128 stays below 2^31.
constexpr int64_t kFullMaxBytes = 0x7FFF0000;

template <int PASS, int D>
__device__ __forceinline__ float ln_pass_full(__amdgpu_buffer_rsrc_t rs, int voff, int nt, int l,
                                              float4 (&tb)[3][64], float mu) {
  static_assert(D % 6 == 0, "LDS buffers rotate by 3, register sets by 2");
  float acc = 0.f;
  v4f_rs buf[D];
#pragma unroll
  for (int u = 0; u < D; u++)
    buf[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + u * 128, 0, 0);
  auto prep = [&](v4f_rs v) {
    float4 o = {v.x, v.y, v.z, v.w};
    if constexpr (PASS != 0) {
      o.x = ln_term<PASS>(o.x, mu);
      o.y = ln_term<PASS>(o.y, mu);
      o.z = ln_term<PASS>(o.z, mu);
      o.w = ln_term<PASS>(o.w, mu);
    }
    return o;
  };
  tb[0][l] = prep(buf[0]);
  tb[1][l] = prep(buf[1]);
  buf[0] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + D * 128, 0, 0);
  buf[1] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + (D + 1) * 128, 0, 0);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // Every lane adds the terms of its row (l & 7): the 8 lanes of a row read
  // the same LDS words (a broadcast) and run the same chain, so no lane
  // masks; the tile being added and the one being read alternate between
  // two register sets by tile parity (D is even), so nothing is copied.
  const int lr = l & 7;
  float4 w[2][8];
#pragma unroll
  for (int q = 0; q < 8; q++) w[0][q] = tb[0][q * 8 + lr];
  for (int t0 = 0; t0 < nt; t0 += D) {
    const int vt = voff + t0 * 128;
#pragma unroll
    for (int u = 0; u < D; u++) {
#pragma unroll
      for (int q = 0; q < 8; q++) w[(u + 1) & 1][q] = tb[(u + 1) % 3][q * 8 + lr];
      tb[(u + 2) % 3][l] = prep(buf[(u + 2) % D]);
      buf[(u + 2) % D] = __builtin_amdgcn_raw_buffer_load_b128(rs, vt + (u + 2 + D) * 128, 0, 0);
      if (t0 + u < nt) {
#pragma unroll
        for (int q = 0; q < 8; q++) {
          acc = acc + w[u & 1][q].x;
          acc = acc + w[u & 1][q].y;
          acc = acc + w[u & 1][q].z;
          acc = acc + w[u & 1][q].w;
        }
      }
      // one wave per workgroup: waiting for its own LDS operations suffices
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
  }
  return acc;
}

// Raw descriptor (stride 0) over `bytes` bytes from p; the last dword sets
// DATA_FORMAT to 32 bits (a zero format would make every load return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, (int)bytes,
                                           0x00020000);
}


}  // namespace rowsum
}  // namespace sdq
