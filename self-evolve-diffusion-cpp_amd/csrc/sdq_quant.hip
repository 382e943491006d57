// Per-row dynamic activation quantizer (gfx950).
//
// Restates src/core/qgemm.cpp:82-96 of the reference bit-exactly:
//   mx  = max_k |A[i,k]|  (NaN inputs never win the max, as std::max(mx,|r|))
//   sc  = mx / 127.f (IEEE, correctly rounded); sc == 0 -> 1
//   inv = 1.f / sc (correctly rounded)
//   q   = clamp(cvt_rne(A[i,k] * inv), -127, 127), where NaN and values whose
//         rounded result leaves int32 give -127 (x86 cvtss2si "indefinite"
//         INT_MIN, then clamped), src/core/qgemm.cpp:62-69.
//
// Every lane loads the 16 floats it will own in a fragment slot (16 bytes of
// one row), keeps up to CACHE such slices in registers across the amax
// reduction (a single HBM read when the row fits), and re-reads only the
// part of the row beyond that. The fragment-layout kernel works on 8-row
// units (a quarter of a fragment row per workgroup) for a fine grid; the
// row-major kernel (parity API) on 32-row blocks. Few long rows take a
// split form instead (per-chunk maxima, then reduce + quantize), so that
// the whole GPU walks them.
#include <cstdlib>

#include "sdq_internal.h"
#include "sdq_device.h"
#include "sdq_rowsum.h"

#pragma clang fp contract(off)

namespace sdq {
namespace {

using dev::quant_one;

constexpr int kQuantWaves = 16;
constexpr int kQuantCache = 6;  // 16 waves x 6 frags x 32 = K <= 3072 in one pass
// Fragment-layout quantizer: 8-row units, 8 waves, 3 fragment groups (of 4
// fragments) cached per lane = K <= 3072 read once (measured 5.2 TB/s at
// M=27280, K=3072 on MI355X vs 3.2 TB/s for whole 32-row fragment rows).
constexpr int kQuantRows = 8;
constexpr int kQuantUnitWaves = 8;
constexpr int kQuantUnitCache = 3;


__device__ __forceinline__ void load16(const float* __restrict__ rowp, int64_t k0, int64_t K,
                                       bool row_ok, bool vec, float v[16]) {
  if (row_ok && vec && k0 + 16 <= K) {
    const float4* p = reinterpret_cast<const float4*>(rowp + k0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 x = p[i];
      v[4 * i + 0] = x.x;
      v[4 * i + 1] = x.y;
      v[4 * i + 2] = x.z;
      v[4 * i + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int64_t k = k0 + e;
      v[e] = (row_ok && k < K) ? rowp[k] : 0.f;
    }
  }
}

__device__ __forceinline__ float amax16(const float v[16], float mx) {
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const float a = fabsf(v[e]);
    mx = (mx < a) ? a : mx;  // std::max(mx, a): keeps mx when a is NaN
  }
  return mx;
}

__device__ __forceinline__ uint4 pack16(const float v[16], float inv) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    uint32_t x = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) x |= (uint32_t)(uint8_t)(int8_t)quant_one(v[4 * i + b], inv) << (8 * b);
    w[i] = x;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Max over c < pc of a row's given maxima pm[c] (pm 16-byte aligned), read
// by the eight lanes l = row + 8j that share the row (lane l takes every
// eighth float4 from l / 8), then combined across them; `ok` (the row
// exists) is the same on all eight. Every lane must call it. NaN never
// enters the maxima, and max is exact and order-free. Each lane issues up
// to eight float4 loads before it uses any (one memory latency for up to
// 256 maxima per row, e.g. a 14336-column fc1's 224, instead of one per
// load); the zeros past the end cannot win, as the maxima are >= 0.
__device__ __forceinline__ float premax_row(const float* __restrict__ pm, int pc, bool ok,
                                            int l) {
  float mx = 0.f;
  if (ok) {
    const float4* p4 = reinterpret_cast<const float4*>(pm);
    const int n4 = pc / 4;
    for (int j0 = l >> 3; j0 < n4; j0 += 64) {
      float4 r[8];
#pragma unroll
      for (int u = 0; u < 8; u++)
        r[u] = j0 + 8 * u < n4 ? p4[j0 + 8 * u] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int u = 0; u < 8; u++) {
        mx = (mx < r[u].x) ? r[u].x : mx;
        mx = (mx < r[u].y) ? r[u].y : mx;
        mx = (mx < r[u].z) ? r[u].z : mx;
        mx = (mx < r[u].w) ? r[u].w : mx;
      }
    }
    for (int j = (pc & ~3) + (l >> 3); j < pc; j += 8) mx = (mx < pm[j]) ? pm[j] : mx;
  }
#pragma unroll
  for (int d = 8; d < 64; d *= 2) {
    const float o = __shfl_xor(mx, d);
    mx = (mx < o) ? o : mx;
  }
  return mx;
}

// mod_rows(layernorm(.)) of 16 consecutive values of one row (columns
// k0 .. k0+15; those >= K are padding and stay 0), the reference build's
// steps: t = fl(v - mu) * inv, rounded; o = t + 0 (-0 -> +0); then
// fmaf(o, 1 + scale[k], shift[k]).
__device__ __forceinline__ void lnmod16(float v[16], int64_t k0, int64_t K, float2 st,
                                        const LnModArgs& lm, bool vec) {
  float sh[16], sc[16];
  if (vec && k0 + 16 <= K) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 a = reinterpret_cast<const float4*>(lm.shift + k0)[i];
      const float4 b = reinterpret_cast<const float4*>(lm.scale + k0)[i];
      sh[4 * i] = a.x; sh[4 * i + 1] = a.y; sh[4 * i + 2] = a.z; sh[4 * i + 3] = a.w;
      sc[4 * i] = b.x; sc[4 * i + 1] = b.y; sc[4 * i + 2] = b.z; sc[4 * i + 3] = b.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 16; e++) {
      sh[e] = k0 + e < K ? lm.shift[k0 + e] : 0.f;
      sc[e] = k0 + e < K ? lm.scale[k0 + e] : 0.f;
    }
  }
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const float d = v[e] - st.x;
    const float t = d * st.y;
    const float o = t + 0.f;
    const float a = 1.f + sc[e];
    const float y = __builtin_fmaf(o, a, sh[e]);
    v[e] = k0 + e < K ? y : 0.f;
  }
}

using rowsum::kFullMaxBytes;
using rowsum::kLnDepthFew;
using rowsum::kLnDepthFull;
using rowsum::kLnDepthMany;
using rowsum::ln_pass;
using rowsum::ln_pass_full;

// Row statistics of blocks.cpp:18-43 (no affine), bit-exact with the
// reference build: the mean and the variance are serial float sums in k
// order (d*d rounded, then added), inv = 1/sqrtf(var/K + eps); two passes
// over the row (mean, then variance).
template <bool VEC, int D>
__global__ void __launch_bounds__(64)
ln_stats_kernel(const float* __restrict__ x, int64_t M, int64_t K, float eps,
                float2* __restrict__ st) {
  __shared__ float4 tb[2][64];
  const int l = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * 8 + (l & 7);
  const bool ok = row < M;
  const float* r = x + (ok ? row : 0) * K;
  float mu = ln_pass<VEC, 0, D>(r, K, l, tb, 0.f);
  mu = mu / (float)K;
  mu = __shfl(mu, l & 7);  // lanes 0-7 hold the rows' sums; lane l works on row l & 7
  const float var = ln_pass<VEC, 1, D>(r, K, l, tb, mu);
  if (l < 8 && ok) {
    const float den = var / (float)K + eps;
    st[row] = float2{mu, 1.f / sqrtf(den)};
  }
}

// The same statistics for K % 32 == 0, 16-byte aligned rows and M*K*4 <=
// kFullMaxBytes: whole 32-column tiles through a buffer descriptor.
__global__ void __launch_bounds__(64)
ln_stats_full_kernel(const float* __restrict__ x, int64_t M, int64_t K, float eps,
                     float2* __restrict__ st) {
  __shared__ float4 tb[3][64];
  const int l = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * 8 + (l & 7);
  const bool ok = row < M;
  const int64_t bytes = M * K * 4;
  const auto rs = rowsum::row_rsrc(x, bytes);
  // rows past M start at the range's end: all their loads return 0
  const int voff = (int)(ok ? (row * K + 4 * (l >> 3)) * 4 : bytes);
  const int nt = (int)(K / 32);
  // every lane holds the sum of its row (l & 7)
  const float mu = ln_pass_full<0, kLnDepthFull>(rs, voff, nt, l, tb, 0.f) / (float)K;
  const float var = ln_pass_full<1, kLnDepthFull>(rs, voff, nt, l, tb, mu);
  if (l < 8 && ok) {
    const float den = var / (float)K + eps;
    st[row] = float2{mu, 1.f / sqrtf(den)};
  }
}

// Row-major output variant (the parity API): one workgroup per 32 rows.
template <int NW, int CACHE, bool FRAG_OUT>
__global__ void __launch_bounds__(NW * 64)
act_quant_kernel(const float* __restrict__ A, int64_t M, int64_t K, int64_t KL, int64_t KFp,
                 int vec, int8_t* __restrict__ out, float* __restrict__ as, ColCopy cc) {
  // Side job: zero-padded copies of the GEMM's per-column bias / gate.
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cc.CP;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (cc.bias_pad) cc.bias_pad[i] = i < cc.N ? cc.bias[i] : 0.f;
    if (cc.gate_pad) cc.gate_pad[i] = i < cc.N ? cc.gate[i] : 0.f;
  }
  const int w = threadIdx.x >> 6;
  const int l = threadIdx.x & 63;
  const int64_t rb = blockIdx.x;
  const int64_t row = rb * 32 + (l & 31);
  const bool row_ok = row < M;
  const float* rowp = A + (row_ok ? row : 0) * K;
  const int kg = (l >> 5) * 16;

  float cache[CACHE][16];
  float mx = 0.f;
#pragma unroll
  for (int c = 0; c < CACHE; c++) {
    const int64_t kb = w + (int64_t)c * NW;
    if (kb < KL) {
      load16(rowp, kb * 32 + kg, K, row_ok, vec != 0, cache[c]);
      mx = amax16(cache[c], mx);
    }
  }
  for (int64_t kb = w + (int64_t)CACHE * NW; kb < KL; kb += NW) {
    float t[16];
    load16(rowp, kb * 32 + kg, K, row_ok, vec != 0, t);
    mx = amax16(t, mx);
  }
  // Lanes l and l^32 hold the same row.
  const float o = __shfl_xor(mx, 32);
  mx = (mx < o) ? o : mx;
  __shared__ float red[NW][32];
  if (l < 32) red[w][l] = mx;
  __syncthreads();
  mx = 0.f;
#pragma unroll
  for (int i = 0; i < NW; i++) {
    const float r = red[i][l & 31];
    mx = (mx < r) ? r : mx;
  }
  float sc = mx / 127.f;
  if (sc == 0.f) sc = 1.f;
  const float inv = 1.f / sc;
  if (w == 0 && l < 32 && row_ok) as[row] = sc;

  auto emit = [&](int64_t kb, const float v[16]) {
    const uint4 q = pack16(v, inv);
    if (FRAG_OUT) {
      *reinterpret_cast<uint4*>(out + (rb * KFp + kb) * 1024 + l * 16) = q;
    } else if (row_ok) {
      const int64_t k0 = kb * 32 + kg;
      int8_t* dst = out + row * K;
      const uint32_t wds[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 16; e++)
        if (k0 + e < K) dst[k0 + e] = (int8_t)(wds[e >> 2] >> (8 * (e & 3)));
    }
  };
#pragma unroll
  for (int c = 0; c < CACHE; c++) {
    const int64_t kb = w + (int64_t)c * NW;
    if (kb < KL) emit(kb, cache[c]);
  }
  for (int64_t kb = w + (int64_t)CACHE * NW; kb < KL; kb += NW) {
    float t[16];
    load16(rowp, kb * 32 + kg, K, row_ok, vec != 0, t);
    emit(kb, t);
  }
}

// Fragment-layout quantizer over R-row units (R = 8 or 16: a quarter or half
// of a fragment row), for a finer grid than one 32-row fragment row per
// workgroup (fewer idle CUs in the last wave of workgroups). Lane l owns
// row unit*R + (l % R), half h = (l / R) & 1 of fragment g*F + l / (2R),
// F = 32 / R fragments per group: the fragment slot (row & 31) + 32h, 16
// bytes, so each fragment is written as two contiguous runs of 16R bytes.
// PRE: the row maxima come from pre[row * pstride + c], c < pc (written by
// the producing GEMM), so the row is read once, with no max pass.
// XF: the quantized rows are mod_rows(layernorm(A)) (ovi_dit.cpp:161-172,
// blocks.cpp:18-43): value v of row r, column k becomes
//   fmaf(fl(fl(v - mu_r) * inv_r) + 0, 1 + scale[k], shift[k])
// with (mu_r, inv_r) from ln_stats_kernel; padding columns stay 0.
// One R-row unit (`unit`) of a quantizer launch.
template <int R, int NW, int CACHE, bool PRE, bool XF>
__device__ __forceinline__ void
act_quant_unit(const float* __restrict__ A, int64_t M, int64_t K, int64_t KFp, int vec,
               int8_t* __restrict__ out, float* __restrict__ as,
               const float* __restrict__ pre, int pc, int pstride, LnModArgs lm,
               const int64_t unit) {
  static_assert(R == 8 || R == 16, "unit height");
  static_assert(!(PRE && XF), "given maxima are for the plain rows");
  constexpr int F = 32 / R;  // fragments per lane group
  const int w = threadIdx.x >> 6;
  const int l = threadIdx.x & 63;
  const int64_t row = unit * R + (l % R);
  const bool row_ok = row < M;
  const float* rowp = A + (row_ok ? row : 0) * K;
  const int sub = l / (2 * R);         // fragment within the group
  const int half = (l / R) & 1;
  const int kg = half * 16;            // k offset inside the fragment
  const int64_t ng = KFp / F;          // fragment groups (KFp is a multiple of 8)
  const int slot = (int)((row & 31) + half * 32) * 16;
  float2 st = {0.f, 0.f};
  if constexpr (XF) st = row_ok ? lm.st[row] : float2{0.f, 0.f};
  // the lane's 16 values of group g (transformed under XF)
  auto fetch = [&](int64_t g, float v[16]) {
    const int64_t k0 = (g * F + sub) * 32 + kg;
    load16(rowp, k0, K, row_ok, vec != 0, v);
    if constexpr (XF) lnmod16(v, k0, K, st, lm, vec != 0);
  };

  float cache[CACHE][16];
  float mx = 0.f;
#pragma unroll
  for (int c = 0; c < CACHE; c++) {
    const int64_t g = w + (int64_t)c * NW;
    if (g < ng) {
      fetch(g, cache[c]);
      if constexpr (!PRE) mx = amax16(cache[c], mx);
    }
  }
  if constexpr (PRE) {
    static_assert(!PRE || R == 8, "given maxima are read by the 8 lanes of a row");
    mx = premax_row(pre + (row_ok ? row : 0) * pstride, pc, row_ok, l);
  } else {
    // (loading several groups per iteration here measured slower at large
    // M: the extra VGPRs cost occupancy, 5 -> 3 waves per SIMD)
    for (int64_t g = w + (int64_t)CACHE * NW; g < ng; g += NW) {
      float t[16];
      fetch(g, t);
      mx = amax16(t, mx);
    }
    // the lanes l + R*j (j = 0 .. 64/R - 1) hold the same row
#pragma unroll
    for (int d = R; d < 64; d *= 2) {
      const float o = __shfl_xor(mx, d);
      mx = (mx < o) ? o : mx;
    }
    __shared__ float red[NW][R];
    if (l < R) red[w][l] = mx;
    __syncthreads();
    mx = 0.f;
#pragma unroll
    for (int i = 0; i < NW; i++) {
      const float r = red[i][l % R];
      mx = (mx < r) ? r : mx;
    }
  }
  float sc = mx / 127.f;
  if (sc == 0.f) sc = 1.f;
  const float inv = 1.f / sc;
  if (w == 0 && l < R && row_ok) as[row] = sc;

  int8_t* base = out + (unit / F) * KFp * 1024 + slot;
  auto emit = [&](int64_t g, const float v[16]) {
    *reinterpret_cast<uint4*>(base + (g * F + sub) * 1024) = pack16(v, inv);
  };
#pragma unroll
  for (int c = 0; c < CACHE; c++) {
    const int64_t g = w + (int64_t)c * NW;
    if (g < ng) emit(g, cache[c]);
  }
  for (int64_t g = w + (int64_t)CACHE * NW; g < ng; g += NW) {
    float t[16];
    fetch(g, t);
    emit(g, t);
  }
}

template <int R, int NW, int CACHE, bool PRE, bool XF>
__global__ void __launch_bounds__(NW * 64)
act_quant_units_kernel(const float* __restrict__ A, int64_t M, int64_t K, int64_t KFp, int vec,
                       int8_t* __restrict__ out, float* __restrict__ as, ColCopy cc,
                       const float* __restrict__ pre, int pc, int pstride, LnModArgs lm) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cc.CP;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (cc.bias_pad) cc.bias_pad[i] = i < cc.N ? cc.bias[i] : 0.f;
    if (cc.gate_pad) cc.gate_pad[i] = i < cc.N ? cc.gate[i] : 0.f;
  }
  act_quant_unit<R, NW, CACHE, PRE, XF>(A, M, K, KFp, vec, out, as, pre, pc, pstride, lm,
                                        blockIdx.x);
}

// Several independent quantizations in one launch (the inputs of Linears
// that do not depend on each other): workgroup b quantizes unit
// b - segs.s[i].unit0 of the segment i whose units it falls in.
__global__ void __launch_bounds__(kQuantUnitWaves * 64)
act_quant_segs_kernel(QuantSegs segs) {
  const int64_t b = blockIdx.x;
  int i = 0;
#pragma unroll
  for (int q = 1; q < kMaxQuantSegs; q++)
    if (q < segs.count && b >= segs.s[q].unit0) i = q;
  const QuantSeg& g = segs.s[i];
  const int64_t unit = b - g.unit0;
  const int64_t units = (i + 1 < segs.count ? segs.s[i + 1].unit0 : segs.total) - g.unit0;
  const ColCopy& cc = g.cc;
  for (int64_t c = unit * blockDim.x + threadIdx.x; c < cc.CP; c += units * blockDim.x) {
    if (cc.bias_pad) cc.bias_pad[c] = c < cc.N ? cc.bias[c] : 0.f;
    if (cc.gate_pad) cc.gate_pad[c] = c < cc.N ? cc.gate[c] : 0.f;
  }
  act_quant_unit<kQuantRows, kQuantUnitWaves, kQuantUnitCache, false, false>(
      g.A, g.M, g.K, g.KFp, g.vec, g.at, g.as, nullptr, 0, 0, LnModArgs{}, unit);
}

// Split form of the fragment-layout quantizer for few rows, where one
// workgroup per 8-row unit walks too much of K serially (latency-bound: a
// handful of workgroups each waiting on dependent row loads). Work item =
// (unit, chunk of GPW fragment groups), one wave each, same lane roles as
// act_quant_units_kernel (R = 8). Pass 1 writes the item's per-row maxima;
// pass 2 reduces a row's maxima (max is exact and order-free; NaN never
// enters, as in amax16) and quantizes its chunk, re-reading it (from L2:
// same grid, so item i runs on the same XCD in both passes).
template <int GPW>
__global__ void __launch_bounds__(256)
act_quant_pmax_kernel(const float* __restrict__ A, int64_t M, int64_t K, int64_t KFp, int vec,
                      int C, int64_t items, float* __restrict__ pmax) {
  constexpr int R = 8, F = 32 / R;
  const int l = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= items) return;
  const int64_t unit = item / C;
  const int c = (int)(item - unit * C);
  const int64_t row = unit * R + (l % R);
  const bool row_ok = row < M;
  const float* rowp = A + (row_ok ? row : 0) * K;
  const int sub = l / (2 * R), kg = ((l / R) & 1) * 16;
  const int64_t ng = KFp / F;
  float v[GPW][16];
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < GPW; i++) {
    const int64_t g = (int64_t)c * GPW + i;
    if (g < ng) {
      load16(rowp, (g * F + sub) * 32 + kg, K, row_ok, vec != 0, v[i]);
      mx = amax16(v[i], mx);
    }
  }
#pragma unroll
  for (int d = R; d < 64; d *= 2) {
    const float o = __shfl_xor(mx, d);
    mx = (mx < o) ? o : mx;
  }
  // rows of pmax have C rounded up to 4 floats (16-byte aligned rows)
  if (l < R) pmax[(unit * R + l) * ((C + 3) & ~3) + c] = mx;
}

template <int GPW>
__global__ void __launch_bounds__(256)
act_quant_emit_kernel(const float* __restrict__ A, int64_t M, int64_t K, int64_t KFp, int vec,
                      int C, int64_t items, const float* __restrict__ pmax, int pc, int pstride,
                      int8_t* __restrict__ out, float* __restrict__ as, ColCopy cc) {
  constexpr int R = 8, F = 32 / R;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cc.CP;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (cc.bias_pad) cc.bias_pad[i] = i < cc.N ? cc.bias[i] : 0.f;
    if (cc.gate_pad) cc.gate_pad[i] = i < cc.N ? cc.gate[i] : 0.f;
  }
  const int l = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= items) return;
  const int64_t unit = item / C;
  const int c = (int)(item - unit * C);
  const int64_t row = unit * R + (l % R);
  const bool row_ok = row < M;
  const float* rowp = A + (row_ok ? row : 0) * K;
  const int sub = l / (2 * R), half = (l / R) & 1, kg = half * 16;
  const int64_t ng = KFp / F;
  float v[GPW][16];
#pragma unroll
  for (int i = 0; i < GPW; i++) {
    const int64_t g = (int64_t)c * GPW + i;
    if (g < ng) load16(rowp, (g * F + sub) * 32 + kg, K, row_ok, vec != 0, v[i]);
  }
  const float mx = premax_row(pmax + (row_ok ? row : 0) * pstride, pc, row_ok, l);
  float sc = mx / 127.f;
  if (sc == 0.f) sc = 1.f;
  const float inv = 1.f / sc;
  if (c == 0 && l < R && row_ok) as[row] = sc;
  int8_t* base = out + (unit / F) * KFp * 1024 + (int)((row & 31) + half * 32) * 16;
#pragma unroll
  for (int i = 0; i < GPW; i++) {
    const int64_t g = (int64_t)c * GPW + i;
    if (g < ng) *reinterpret_cast<uint4*>(base + (g * F + sub) * 1024) = pack16(v[i], inv);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Fragment groups per split item: 4 from 64 units up (measured at K=14336:
// M=512 16.3 vs 19.0 us, M=768 22.1 vs 25.2), else 2 (M=157 12.7 vs 14.4).
int split_gpw(int64_t Mp) { return Mp / kQuantRows >= 64 ? 4 : 2; }
int64_t split_chunks(int64_t Mp, int64_t KFp) {
  return ceil_div(KFp / (32 / kQuantRows), split_gpw(Mp));
}

}  // namespace

// The split form pays a second launch and a re-read from L2; it wins for
// long rows (several times the single kernel's register cache) in few 8-row
// units. Measured (single vs split, us): K=14336: M=157 30.5 / 12.7, M=768
// 31.3 / 22.1, M=2048 36.1 / 44.6; K=8192: M=157 18.0 / 9.6, M=768 17.2 /
// 15.0, M=2048 24.3 / 28.0; K=6144: M=157 14.3 / 9.9, M=512 13.2 / 12.2,
// M=768 13.8 / 15.2; K=4096: M=512 10.6 / 12.9; K=3072: M=157 7.4 / 9.1.
// (cu_count scales the unit limits from the 256-CU part.)
bool split_wins(int64_t units, int64_t KFp, int cu_count) {
  const int64_t c = cu_count > 0 ? cu_count : 256;
  if (KFp >= 256) return units * 2 < c;  // K >= 8192: M < 1024
  if (KFp >= 192) return units * 4 <= c;  // K >= 6144: M <= 512
  return false;
}

int64_t act_quant_pmax_floats(int64_t Mp, int64_t KFp, int cu_count) {
  // SDQ_QUANT_SINGLE forces the single kernel, for comparisons.
  if (std::getenv("SDQ_QUANT_SINGLE")) return 0;
  return split_wins(Mp / kQuantRows, KFp, cu_count) ? Mp * ((split_chunks(Mp, KFp) + 3) & ~3) : 0;
}

hipError_t launch_act_quant_frags(const float* A, int64_t M, int64_t K, int64_t Mp, int64_t KFp,
                                  int8_t* at, float* as, const ColCopy& cc, float* pmax,
                                  int cu_count, hipStream_t s) {
  const int vec = (aligned16(A) && (K % 4) == 0) ? 1 : 0;
  const int64_t units = Mp / kQuantRows;
  if (pmax && act_quant_pmax_floats(Mp, KFp, cu_count) > 0) {
    const int C = (int)split_chunks(Mp, KFp), Cp = (C + 3) & ~3;
    const int64_t items = units * C;
    const unsigned blocks = (unsigned)ceil_div(items, 4);
    if (split_gpw(Mp) == 4) {
      hipLaunchKernelGGL((act_quant_pmax_kernel<4>), dim3(blocks), dim3(256), 0, s, A, M, K, KFp,
                         vec, C, items, pmax);
      hipLaunchKernelGGL((act_quant_emit_kernel<4>), dim3(blocks), dim3(256), 0, s, A, M, K, KFp,
                         vec, C, items, pmax, C, Cp, at, as, cc);
    } else {
      hipLaunchKernelGGL((act_quant_pmax_kernel<2>), dim3(blocks), dim3(256), 0, s, A, M, K, KFp,
                         vec, C, items, pmax);
      hipLaunchKernelGGL((act_quant_emit_kernel<2>), dim3(blocks), dim3(256), 0, s, A, M, K, KFp,
                         vec, C, items, pmax, C, Cp, at, as, cc);
    }
    return hipGetLastError();
  }
  hipLaunchKernelGGL((act_quant_units_kernel<kQuantRows, kQuantUnitWaves, kQuantUnitCache, false, false>),
                     dim3((unsigned)units), dim3(kQuantUnitWaves * 64), 0, s, A, M, K, KFp, vec,
                     at, as, cc, nullptr, 0, 0, LnModArgs{});
  return hipGetLastError();
}

hipError_t launch_act_quant_segs(const QuantSegs& segs, hipStream_t s) {
  if (segs.count < 1 || segs.count > kMaxQuantSegs || segs.total <= 0 ||
      segs.total > 0x7FFFFFFF)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(act_quant_segs_kernel, dim3((unsigned)segs.total),
                     dim3(kQuantUnitWaves * 64), 0, s, segs);
  return hipGetLastError();
}

hipError_t launch_ln_stats(const float* A, int64_t M, int64_t K, float eps, float2* st,
                           hipStream_t s) {
  if (M <= 0) return hipSuccess;
  if (K <= 0 || !st) return hipErrorInvalidValue;
  const bool vx = aligned16(A) && (K % 4) == 0, few = M <= 4096;
  const dim3 g((unsigned)ceil_div(M, 8)), b(64);
  if (vx && K % 32 == 0 && M * K * 4 <= kFullMaxBytes)
    hipLaunchKernelGGL(ln_stats_full_kernel, g, b, 0, s, A, M, K, eps, st);
  else if (vx && few)
    hipLaunchKernelGGL((ln_stats_kernel<true, kLnDepthFew>), g, b, 0, s, A, M, K, eps, st);
  else if (vx)
    hipLaunchKernelGGL((ln_stats_kernel<true, kLnDepthMany>), g, b, 0, s, A, M, K, eps, st);
  else if (few)
    hipLaunchKernelGGL((ln_stats_kernel<false, kLnDepthFew>), g, b, 0, s, A, M, K, eps, st);
  else
    hipLaunchKernelGGL((ln_stats_kernel<false, kLnDepthMany>), g, b, 0, s, A, M, K, eps, st);
  return hipGetLastError();
}

hipError_t launch_act_quant_frags_lnmod(const float* A, int64_t M, int64_t K, int64_t Mp,
                                        int64_t KFp, int8_t* at, float* as, const ColCopy& cc,
                                        const float* shift, const float* scale, float eps,
                                        float2* st, hipStream_t s) {
  if (!shift || !scale || !st || K <= 0) return hipErrorInvalidValue;
  const int vec = (aligned16(A) && aligned16(shift) && aligned16(scale) && (K % 4) == 0) ? 1 : 0;
  hipError_t e = launch_ln_stats(A, M, K, eps, st, s);
  if (e != hipSuccess) return e;
  const int64_t units = Mp / kQuantRows;
  LnModArgs lm{st, shift, scale};
  hipLaunchKernelGGL((act_quant_units_kernel<kQuantRows, kQuantUnitWaves, kQuantUnitCache, false, true>),
                     dim3((unsigned)units), dim3(kQuantUnitWaves * 64), 0, s, A, M, K, KFp, vec,
                     at, as, cc, nullptr, 0, 0, lm);
  return hipGetLastError();
}

hipError_t launch_act_quant_frags_premax(const float* A, int64_t M, int64_t K, int64_t Mp,
                                         int64_t KFp, int8_t* at, float* as, const ColCopy& cc,
                                         const float* rmax, int rchunks, int rstride,
                                         int cu_count, hipStream_t s) {
  if (!rmax || rchunks < 1 || rstride < rchunks || (rstride & 3) || !aligned16(rmax))
    return hipErrorInvalidValue;
  const int vec = (aligned16(A) && (K % 4) == 0) ? 1 : 0;
  const int64_t units = Mp / kQuantRows;
  // Few long rows: the split form's second kernel alone, over the whole GPU.
  if (split_wins(units, KFp, cu_count)) {
    const int C = (int)split_chunks(Mp, KFp);
    const int64_t items = units * C;
    const unsigned blocks = (unsigned)ceil_div(items, 4);
    if (split_gpw(Mp) == 4)
      hipLaunchKernelGGL((act_quant_emit_kernel<4>), dim3(blocks), dim3(256), 0, s, A, M, K, KFp,
                         vec, C, items, rmax, rchunks, rstride, at, as, cc);
    else
      hipLaunchKernelGGL((act_quant_emit_kernel<2>), dim3(blocks), dim3(256), 0, s, A, M, K, KFp,
                         vec, C, items, rmax, rchunks, rstride, at, as, cc);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((act_quant_units_kernel<kQuantRows, kQuantUnitWaves, kQuantUnitCache, true, false>),
                     dim3((unsigned)units), dim3(kQuantUnitWaves * 64), 0, s, A, M, K, KFp, vec,
                     at, as, cc, rmax, rchunks, rstride, LnModArgs{});
  return hipGetLastError();
}

hipError_t launch_act_quant_rowmajor(const float* A, int64_t M, int64_t K, int8_t* aq, float* as,
                                     hipStream_t s) {
  const int vec = (aligned16(A) && (K % 4) == 0) ? 1 : 0;
  const int64_t blocks = ceil_div(M, kFragRows);
  const int64_t KL = ceil_div(K, kFragK);
  hipLaunchKernelGGL((act_quant_kernel<kQuantWaves, kQuantCache, false>), dim3((unsigned)blocks),
                     dim3(kQuantWaves * 64), 0, s, A, M, K, KL, KL, vec, aq, as, ColCopy{});
  return hipGetLastError();
}

}  // namespace sdq
