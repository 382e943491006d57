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

#include <cstdlib>
#include <type_traits>
#include "sdq_rowsum.h"

#pragma clang fp contract(off)

namespace sdq {
namespace {

using rowsum::kFullMaxBytes;
using rowsum::kLnDepthFew;
using rowsum::kLnDepthFull;
using rowsum::kLnDepthMany;
using rowsum::ln_pass;
using rowsum::ln_pass_full;

// Up to kMaxRmsSegs column blocks of strided rows in one launch (e.g. the q
// and k blocks of q|k|v, or cross q, context k and fusion k): their serial
// row sums run side by side instead of one chain after the other.
struct RmsSegs {
  RmsSeg s[kMaxRmsSegs];
  int64_t blk0[kMaxRmsSegs + 1];   // first stats block (8 rows each) of segment i
  int64_t item0[kMaxRmsSegs + 1];  // first apply item (one pair each) of segment i
  int n;
};

__device__ __forceinline__ int seg_of(const int64_t* start, int n, int64_t v) {
  int i = 0;
#pragma unroll
  for (int k = 1; k < kMaxRmsSegs; k++)
    if (k < n && v >= start[k]) i = k;
  return i;
}

// inv[row] = 1/sqrtf(sum_k fl(x[row,k]^2)/C + eps), rows of stride ld.
template <bool VEC, int D>
__global__ void __launch_bounds__(64)
rms_stats_kernel(RmsSegs sg, int64_t C, float eps) {
  __shared__ float4 tb[2][64];
  const int l = threadIdx.x;
  const int i = seg_of(sg.blk0, sg.n, (int64_t)blockIdx.x);
  const RmsSeg& g = sg.s[i];
  const int64_t row = ((int64_t)blockIdx.x - sg.blk0[i]) * 8 + (l & 7);
  const bool ok = row < g.L;
  const float* r = g.x + (ok ? row : 0) * g.ld;
  const float ss = ln_pass<VEC, 2, D>(r, C, l, tb, 0.f);
  if (l < 8 && ok) {
    const float den = ss / (float)C + eps;
    g.inv[row] = 1.f / sqrtf(den);
  }
}

// Bytes the segment's rows span: (L-1) strides and one row of C.
__host__ __device__ inline int64_t seg_span_bytes(const RmsSeg& g, int64_t C) {
  return ((g.L - 1) * g.ld + C) * 4;
}

// The same statistics when every segment has C % 32 == 0, 16-byte aligned
// rows and a span of at most kFullMaxBytes: whole 32-column tiles through a
// buffer descriptor over the segment's rows.
__global__ void __launch_bounds__(64)
rms_stats_full_kernel(RmsSegs sg, int64_t C, float eps) {
  __shared__ float4 tb[3][64];
  const int l = threadIdx.x;
  const int i = seg_of(sg.blk0, sg.n, (int64_t)blockIdx.x);
  const RmsSeg& g = sg.s[i];
  const int64_t row = ((int64_t)blockIdx.x - sg.blk0[i]) * 8 + (l & 7);
  const bool ok = row < g.L;
  const int64_t bytes = seg_span_bytes(g, C);
  const auto rs = rowsum::row_rsrc(g.x, bytes);
  // rows past L start at the range's end: all their loads return 0
  const int voff = (int)(ok ? (row * g.ld + 4 * (l >> 3)) * 4 : bytes);
  const float ss = ln_pass_full<2, kLnDepthFull>(rs, voff, (int)(C / 32), l, tb, 0.f);
  if (l < 8 && ok) {
    const float den = ss / (float)C + eps;
    g.inv[row] = 1.f / sqrtf(den);
  }
}

// y = fl(fl(v*inv)*w) over the row, then the rotation of each head's first
// nr pairs. One thread per pair (pairs never straddle heads: hd is even);
// grid.y is the segment, so its fields are wave-uniform. IDX32: the
// segment's L*C/2 pairs fit 32-bit index math.
template <bool IDX32>
__global__ void __launch_bounds__(256)
rms_rope_apply_kernel(RmsSegs sg, int64_t C, int hd) {
  const RmsSeg& g = sg.s[blockIdx.y];
  const int64_t np = C / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= g.L * np) return;
  int64_t row, p;
  if constexpr (IDX32) {
    const uint32_t r32 = (uint32_t)idx / (uint32_t)np;
    row = r32;
    p = (int64_t)((uint32_t)idx - r32 * (uint32_t)np);
  } else {
    row = idx / np;
    p = idx - row * np;
  }
  const int64_t c0 = 2 * p;
  float* q = g.x + row * g.ld + c0;
  float y0 = q[0], y1 = q[1];
  if (g.w) {
    const float iv = g.inv[row];
    const float a = y0 * iv, b = y1 * iv;
    y0 = a * g.w[c0];
    y1 = b * g.w[c0 + 1];
  }
  const int j = (int)(c0 % hd) / 2;  // pair index inside the head
  if (g.cs && j < g.nr) {
    const float2 t = reinterpret_cast<const float2*>(g.cs)[row * g.nr + j];  // (cos, sin)
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

hipError_t launch_rmsnorm_rope_segs(const RmsSeg* segs, int nseg, int64_t C, int heads, float eps,
                                    hipStream_t s) {
  if (nseg < 1 || nseg > kMaxRmsSegs || C <= 0 || heads <= 0 || C % heads || (C / heads) % 2)
    return hipErrorInvalidValue;
  RmsSegs st{};
  st.n = nseg;
  bool vec = C % 4 == 0, few = true, any_w = false, full = C % 32 == 0;
  for (int i = 0; i < nseg; i++) {
    const RmsSeg& g = segs[i];
    if (g.L < 0 || g.ld < C || g.nr < 0 || g.nr > C / heads / 2 || (!g.w && !g.cs) ||
        (g.w && !g.inv) || (g.L > 0 && !g.x))
      return hipErrorInvalidValue;
    st.s[i] = g;
    st.blk0[i + 1] = st.blk0[i] + (g.w ? ceil_div(g.L, 8) : 0);
    st.item0[i + 1] = st.item0[i] + g.L * (C / 2);
    vec = vec && aligned16(g.x) && g.ld % 4 == 0;
    few = few && g.L <= 4096;
    any_w = any_w || (g.w && g.L > 0);
    full = full && (g.L == 0 || seg_span_bytes(g, C) <= kFullMaxBytes);
  }
  full = full && vec;
  // segments without a weight (rotation only) own no stats blocks
  if (any_w) {
    const dim3 g((unsigned)st.blk0[nseg]), b(64);
    if (full)
      hipLaunchKernelGGL(rms_stats_full_kernel, g, b, 0, s, st, C, eps);
    else if (vec && few)
      hipLaunchKernelGGL((rms_stats_kernel<true, kLnDepthFew>), g, b, 0, s, st, C, eps);
    else if (vec)
      hipLaunchKernelGGL((rms_stats_kernel<true, kLnDepthMany>), g, b, 0, s, st, C, eps);
    else if (few)
      hipLaunchKernelGGL((rms_stats_kernel<false, kLnDepthFew>), g, b, 0, s, st, C, eps);
    else
      hipLaunchKernelGGL((rms_stats_kernel<false, kLnDepthMany>), g, b, 0, s, st, C, eps);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  int64_t most = 0;  // pairs of the largest segment
  for (int i = 0; i < nseg; i++) most = most > segs[i].L * (C / 2) ? most : segs[i].L * (C / 2);
  if (most == 0) return hipSuccess;
  const dim3 ga((unsigned)ceil_div(most, 256), (unsigned)nseg);
  if (most < (int64_t)1 << 31)
    hipLaunchKernelGGL((rms_rope_apply_kernel<true>), ga, dim3(256), 0, s, st, C, (int)(C / heads));
  else
    hipLaunchKernelGGL((rms_rope_apply_kernel<false>), ga, dim3(256), 0, s, st, C, (int)(C / heads));
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rope(float* x, int64_t L, int64_t C, int64_t ld, const float* w,
                               float eps, int heads, const float* cs, int nr, float* inv,
                               hipStream_t s) {
  if (L <= 0) return hipSuccess;
  const RmsSeg g{x, L, ld, w, cs, nr, inv};
  return launch_rmsnorm_rope_segs(&g, 1, C, heads, eps, s);
}


namespace {

__global__ void __launch_bounds__(256)
ln_apply_kernel(const float* x, int64_t M, int64_t K, const float2* __restrict__ st,
                const float* __restrict__ w, const float* __restrict__ b, float* y) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * K) return;
  const int64_t row = idx / K, k = idx - row * K;
  const float2 s2 = st[row];
  const float d = x[idx] - s2.x;
  const float t = d * s2.y;
  y[idx] = __builtin_fmaf(t, w ? w[k] : 1.f, b ? b[k] : 0.f);
}

__global__ void __launch_bounds__(256)
add_kernel(float* x, const float* y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = x[i] + y[i];
}

typedef float v4f_t __attribute__((ext_vector_type(4)));

// The residual step as the GEMM epilogue applies it (contraction is off
// outside the explicit fma).
__device__ __forceinline__ float resid_apply(float x, float y, float g, int kind, int fma) {
  if (kind == SDQ_EPI_RESID) return x + y;
  return fma ? __builtin_fmaf(y, g, x) : x + y * g;
}

// Four consecutive columns per thread: i indexes float4 groups of x.
__global__ void __launch_bounds__(256)
resid2_kernel(float* __restrict__ x, int64_t n4, int64_t N4, ResidStep a, ResidStep b) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const int64_t c = i % N4;
  v4f_t v = reinterpret_cast<const v4f_t*>(x)[i];
  const v4f_t ya = reinterpret_cast<const v4f_t*>(a.y)[i];
  const v4f_t yb = reinterpret_cast<const v4f_t*>(b.y)[i];
  const v4f_t ga = a.gate ? reinterpret_cast<const v4f_t*>(a.gate)[c] : v4f_t{0.f, 0.f, 0.f, 0.f};
  const v4f_t gb = b.gate ? reinterpret_cast<const v4f_t*>(b.gate)[c] : v4f_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float t = resid_apply(v[e], ya[e], ga[e], a.kind, a.gate_fma);
    v[e] = resid_apply(t, yb[e], gb[e], b.kind, b.gate_fma);
  }
  reinterpret_cast<v4f_t*>(x)[i] = v;
}

}  // namespace

hipError_t launch_ln_apply(const float* x, int64_t M, int64_t K, const float2* st, const float* w,
                           const float* b, float* y, hipStream_t s) {
  const int64_t n = M * K;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(ln_apply_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, x, M, K,
                     st, w, b, y);
  return hipGetLastError();
}

hipError_t launch_add(float* x, const float* y, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(add_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

hipError_t launch_resid2(float* x, int64_t M, int64_t N, const ResidStep& a, const ResidStep& b,
                         hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  auto ok = [](int k) { return k == SDQ_EPI_GATED || k == SDQ_EPI_RESID; };
  if (N % 4 != 0 || !ok(a.kind) || !ok(b.kind) || !a.y || !b.y ||
      (a.kind == SDQ_EPI_GATED && !a.gate) || (b.kind == SDQ_EPI_GATED && !b.gate))
    return hipErrorInvalidValue;
  const int64_t n4 = M * N / 4;
  hipLaunchKernelGGL(resid2_kernel, dim3((unsigned)ceil_div(n4, 256)), dim3(256), 0, s, x, n4,
                     N / 4, a, b);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Scaled dot-product attention (src/model/blocks.cpp:112-199, non-causal):
// out[i, head] = softmax_j(q_i . k_j / sqrt(hd)) v_j, head_dim 128: the
// scores as three fp16 products per fp32 product on v_mfma_f32_32x32x16_f16
// (the softmax's exponential would amplify any error in them: each q and k
// row is scaled by a power of two into [0.5, 1) of its largest element, then
// split as x = hi + lo, hi = fp16(x), lo = fp16(x - hi), and q.k taken as
// hi.hi + hi.lo + lo.hi, ~2^-22 relative per product; the powers of two come
// back out exactly in fp32), P.V as three bf16 products per fp32 product on
// v_mfma_f32_32x32x16_bf16 (~2^-17 relative, P in [0, 1]), an online softmax
// (running max and sum per query, the accumulator rescaled when the max
// moves), fp32 accumulation. The reference sums in a fixed serial order, so
// results agree within 2e-5 of the output scale, not bit for bit.
//
// Work: a workgroup of NW waves takes 32*NW queries of one head; each wave
// 32 queries. Per 32-key block, K (32 x 128) and V^T (128 x 32) are staged
// in LDS (double-buffered, prefetched through registers) and every wave
//   S^T = K . Q^T    32 keys x 32 queries: lane (query j = l & 31, half
//                    h = l >> 5) holds 16 keys of its query, so the softmax
//                    of a query is one lane plus its partner lane l ^ 32;
//                    MFMA step s takes dims 64h + 8s .. +7 in both operands
//                    (Q's fp16 parts stay in 64 VGPRs, K's are read 16 bytes
//                    at a time); each key's score is then multiplied by its
//                    row's power of two, the query's goes into the softmax's
//                    scale.
//   O^T += V^T . P^T 128 dims x 32 queries in four 32 x 32 tiles; step t's
//                    key in half h is 8(t/4) + 4h + t%4, exactly the key of
//                    the lane's S^T register t, so P feeds the MFMA with no
//                    shuffle.
// Software pipeline: the scores of block kb+1 are issued before the softmax
// of block kb, so the MFMA pipe works while the wave runs the softmax; K runs
// one block ahead of V in LDS (K of kb+2 and V of kb+1 are written at the end
// of iteration kb, into buffers last read before the previous barrier), so
// one barrier per block suffices.
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
constexpr int kHd = 128;      // head dim
constexpr int kKB = 32;       // keys per block
constexpr int kKPadH = 136;   // LDS row of K's fp16 parts (halves): conflict-free 16-byte reads
constexpr int kVPd = 20;      // LDS row of V^T (dwords: 32 bf16 + pad; conflict-free stash)

// Key split (SPLIT): workgroup z of the grid takes key blocks [z*kbs,
// (z+1)*kbs) and writes its unnormalized output and its (max, sum) state to
// part (layout in SdpaPart); sdpa_merge_kernel combines the splits.
struct SdpaPart {
  float* o;    // [splits][rows][heads * 128]: unnormalized sum of p * v
  float2* ml;  // [splits][rows][heads]: (running max, sum of p), base 2
  int64_t rows;  // batch * Lq
  int heads;
  int kbs;     // key blocks per split
};

// Exponent e with x * 2^-e in [0.5, 1) for a row's largest magnitude x
// (0 for a zero row, so its factor is 1).
__device__ __forceinline__ int row_exp(float x) {
  return x > 0.f && x <= 3.4e38f ? __builtin_amdgcn_frexp_expf(x) : 0;
}

// x = hi + lo + O(2^-22 |x|) in fp16 (|x| < 1 here: no overflow)
struct HalfPair {
  _Float16 hi, lo;
};
__device__ __forceinline__ HalfPair split_f16(float x) {
  const _Float16 hi = (_Float16)x;
  return HalfPair{hi, (_Float16)(x - (float)hi)};
}

// max / sum of a lane's value and lane l ^ 32's, in both lanes (one VALU
// lane swap instead of an LDS permute)
__device__ __forceinline__ float pair32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// max over the 32 lanes of each half-wave, in all of them: DPP within rows of
// 16 (xor 1, xor 2, then the half-row and row mirrors pair the reduced
// groups), then a row swap pairs rows 0-1 and 2-3
__device__ __forceinline__ float half_wave_max(float v) {
  auto dpp = [](float x, auto ctrl_tag) {
    constexpr int ctrl = decltype(ctrl_tag)::value;
    return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), ctrl, 0xF, 0xF,
                                                       false));
  };
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm 1,0,3,2
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm 2,3,0,1
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x141>{}));  // row_half_mirror
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row_mirror
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <int NW, bool SPLIT>
__global__ void __launch_bounds__(NW * 64)
sdpa_kernel(const float* __restrict__ Q, int64_t ldq, const float* __restrict__ K, int64_t ldk,
            const float* __restrict__ V, int64_t ldv, float* __restrict__ O, int64_t ldo,
            int64_t Lq, int64_t Lk, int qgroups, float scale_log2e, SdpaPart part) {
  // Sequence blockIdx.y of a batch: its Lq query rows and Lk key rows follow
  // the previous sequence's (stacked rows, attention stays inside each).
  Q += (int64_t)blockIdx.y * Lq * ldq;
  O += (int64_t)blockIdx.y * Lq * ldo;
  K += (int64_t)blockIdx.y * Lk * ldk;
  V += (int64_t)blockIdx.y * Lk * ldv;
  // K as fp16 hi and lo parts of each row scaled by 2^-e (its largest
  // element in [0.5, 1)); 2^e per key in a ring of three blocks (a block's
  // factors are read in the iteration after its K buffer was refilled)
  __shared__ __attribute__((aligned(16))) _Float16 ksh[2][kKB][kKPadH];
  __shared__ __attribute__((aligned(16))) _Float16 ksl[2][kKB][kKPadH];
  __shared__ __attribute__((aligned(16))) float kexp[3][kKB];
  // V^T as bf16 hi and lo parts, two keys per dword, keys of each 16-key
  // group stored in the order 0-3, 8-11, 4-7, 12-15 (lane half h then reads
  // its 8 keys of a PV step as one 16-byte run)
  __shared__ __attribute__((aligned(16))) uint32_t vth[2][kHd][kVPd];
  __shared__ __attribute__((aligned(16))) uint32_t vtl[2][kHd][kVPd];
  constexpr int NT = NW * 64;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int head = blockIdx.x / qgroups, qg = blockIdx.x - head * qgroups;
  const int64_t q0 = ((int64_t)qg * NW + w) * 32;
  const int j = lane & 31, h = lane >> 5;
  const int64_t col = (int64_t)head * kHd;
  // key blocks of this workgroup: all, or its split's range
  int64_t kb0 = 0;
  if constexpr (SPLIT) kb0 = (int64_t)blockIdx.z * part.kbs;

  // this lane's query row, dims 64h .. 64h+63, scaled by 2^-e (the row's
  // largest element in [0.5, 1)) and split into fp16 parts for the 8 MFMA
  // steps; sq = scale * log2(e) * 2^e puts the factor back in the softmax
  v8h qh[8], ql[8];
  float sq;
  {
    const int64_t qi = q0 + j;
    const float* src = Q + (qi < Lq ? qi : 0) * ldq + col + 64 * h;
    float qr[64];
    float mq = 0.f;
#pragma unroll
    for (int c = 0; c < 16; c++) {
      const float4 v = qi < Lq ? reinterpret_cast<const float4*>(src)[c] : float4{0.f, 0.f, 0.f, 0.f};
      qr[4 * c] = v.x;
      qr[4 * c + 1] = v.y;
      qr[4 * c + 2] = v.z;
      qr[4 * c + 3] = v.w;
      mq = fmaxf(mq, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    mq = pair32_max(mq);
    const int eq = row_exp(mq);
    sq = ldexpf(scale_log2e, eq);
#pragma unroll
    for (int st8 = 0; st8 < 8; st8++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const HalfPair p = split_f16(ldexpf(qr[8 * st8 + e], -eq));
        qh[st8][e] = p.hi;
        ql[st8][e] = p.lo;
      }
  }
  // Cooperative block loads. K: 32 keys x 32 float4, element f is (key
  // f >> 5, float4 f & 31), whole rows per half-wave. V: 16 key pairs x 32
  // float4s, item f is (pair f & 15, float4 2(f >> 5) + ((f >> 4) & 1)); a
  // pair is the two keys that share a dword of the stored order, so the
  // stash writes packed bf16x2 dwords, 32 distinct banks per half-wave.
  // Blocks past the end load zeros.
  constexpr int PER = (kKB * kHd / 4 + NT - 1) / NT;
  static_assert(PER * NT == kKB * kHd / 4, "every lane stashes whole K row slots (half-wave rows)");
  constexpr int PERV = (kKB / 2 * kHd / 4 + NT - 1) / NT;
  float4 pk[PER], pv0[PERV], pv1[PERV];
  // stored position p (0..31) -> key: quads 1 and 2 of each 16 swapped
  auto pos_key = [](int p) {
    const int q = (p >> 2) & 3;
    return (p & 16) + (q == 1 ? 8 : q == 2 ? 4 : 4 * q) + (p & 3);
  };
  auto fetch_k = [&](int64_t kb) {
    if constexpr (SPLIT) kb += kb0;
#pragma unroll
    for (int c = 0; c < PER; c++) {
      const int f = tid + c * NT;
      const int64_t kr = kb * kKB + (f >> 5);
      pk[c] = f < kKB * kHd / 4 && kr < Lk
                  ? *reinterpret_cast<const float4*>(K + kr * ldk + col + 4 * (f & 31))
                  : float4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto fetch_v = [&](int64_t kb) {
    if constexpr (SPLIT) kb += kb0;
#pragma unroll
    for (int c = 0; c < PERV; c++) {
      const int f = tid + c * NT;
      const int kp = f & 15, d4 = 2 * (f >> 5) + ((f >> 4) & 1);
      const int64_t k0 = kb * kKB + pos_key(2 * kp), k1 = kb * kKB + pos_key(2 * kp + 1);
      const bool okf = f < kKB / 2 * kHd / 4;
      pv0[c] = okf && k0 < Lk ? *reinterpret_cast<const float4*>(V + k0 * ldv + col + 4 * d4)
                              : float4{0.f, 0.f, 0.f, 0.f};
      pv1[c] = okf && k1 < Lk ? *reinterpret_cast<const float4*>(V + k1 * ldv + col + 4 * d4)
                              : float4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // K block into buffer b, its keys' factors into ring slot `slot`: the 32
  // lanes of a half-wave hold one key row (PER * NT = 32 * 32 float4s), so
  // the row's largest element is a 32-lane reduction
  auto stash_k = [&](int b, int slot) {
#pragma unroll
    for (int c = 0; c < PER; c++) {
      const int f = tid + c * NT;
      const float4 v = pk[c];
      const float mk =
          half_wave_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
      const int ek = row_exp(mk);
      const HalfPair px = split_f16(ldexpf(v.x, -ek)), py = split_f16(ldexpf(v.y, -ek));
      const HalfPair pz = split_f16(ldexpf(v.z, -ek)), pw = split_f16(ldexpf(v.w, -ek));
      const v4h hi = {px.hi, py.hi, pz.hi, pw.hi}, lo = {px.lo, py.lo, pz.lo, pw.lo};
      *reinterpret_cast<v4h*>(&ksh[b][f >> 5][4 * (f & 31)]) = hi;
      *reinterpret_cast<v4h*>(&ksl[b][f >> 5][4 * (f & 31)]) = lo;
      if ((f & 31) == 0) kexp[slot][f >> 5] = ldexpf(1.f, ek);
    }
  };
  // x -> (bf16(x), bf16(x - bf16(x))) for the two keys of a dword
  auto split2 = [](float x0, float x1, uint32_t& hi, uint32_t& lo) {
    const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
    const __bf16 l0 = (__bf16)(x0 - (float)h0), l1 = (__bf16)(x1 - (float)h1);
    hi = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
    lo = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
  };
  auto stash_v = [&](int b) {
#pragma unroll
    for (int c = 0; c < PERV; c++) {
      const int f = tid + c * NT;
      if (f < kKB / 2 * kHd / 4) {
        const int kp = f & 15, d = 4 * (2 * (f >> 5) + ((f >> 4) & 1));
        const float a0[4] = {pv0[c].x, pv0[c].y, pv0[c].z, pv0[c].w};
        const float a1[4] = {pv1[c].x, pv1[c].y, pv1[c].z, pv1[c].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          uint32_t hi, lo;
          split2(a0[e], a1[e], hi, lo);
          vth[b][d + e][kp] = hi;
          vtl[b][d + e][kp] = lo;
        }
      }
    }
  };
  // S^T = K . Q^T (keys x queries, both scaled) from K buffer b: per step
  // hi.hi + hi.lo + lo.hi
  auto scores = [&](int b) {
    v16f st = v16f{};
    const _Float16* khrow = &ksh[b][j][64 * h];
    const _Float16* klrow = &ksl[b][j][64 * h];
#pragma unroll
    for (int s8 = 0; s8 < 8; s8++) {
      const v8h kh = *reinterpret_cast<const v8h*>(khrow + 8 * s8);
      const v8h kl = *reinterpret_cast<const v8h*>(klrow + 8 * s8);
      st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[s8], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, ql[s8], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[s8], st, 0, 0, 0);
    }
    return st;
  };

  v16f acc[4];
#pragma unroll
  for (int t = 0; t < 4; t++) acc[t] = v16f{};
  float m = -INFINITY, lsum = 0.f;
  int64_t nkb = (Lk + kKB - 1) / kKB;
  if constexpr (SPLIT) nkb = (nkb - kb0) < part.kbs ? (nkb - kb0) : part.kbs;
  // prologue: K(0) -> scores; then K(1) and V(0) staged
  fetch_k(0);
  stash_k(0, 0);
  fetch_k(1);
  fetch_v(0);
  __syncthreads();
  v16f st = scores(0);
  stash_k(1, 1);
  stash_v(0);
  __syncthreads();
  for (int64_t kb = 0; kb < nkb; kb++) {
    const int b = (int)(kb & 1);
    fetch_k(kb + 2);
    fetch_v(kb + 1);
    // scores of the next block (discarded after the last block)
    const v16f sn = scores(b ^ 1);
    // online softmax (base 2, m in units of scale*log2 e) of this block:
    // register r holds key kb*32 + 8(r/4) + 4h + r%4 (times its row factor
    // 2^-e_k, put back here); keys past Lk are -inf.
    // v_exp_f32 flushes results below 2^-126 to 0, which moves a row sum
    // that holds a 1 (the max) by less than 2^-121.
    const int64_t kba = SPLIT ? kb0 + kb : kb;  // the block's index among all keys
    const int rem = Lk - kba * kKB < kKB ? (int)(Lk - kba * kKB) : kKB;
    float t[16];
    float mloc = -INFINITY;
    const float* kf = kexp[(int)(kb % 3)];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const float4 f4 = *reinterpret_cast<const float4*>(kf + 8 * g + 4 * h);
      const float fg[4] = {f4.x, f4.y, f4.z, f4.w};
#pragma unroll
      for (int r = 4 * g; r < 4 * g + 4; r++) t[r] = st[r] * fg[r & 3];
    }
    // only a last, partial block has keys to mask (a uniform branch)
    if (rem < kKB) {
#pragma unroll
      for (int r = 0; r < 16; r++)
        if (8 * (r >> 2) + 4 * h + (r & 3) >= rem) t[r] = -INFINITY;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) mloc = fmaxf(mloc, t[r]);
    const float mnew = fmaxf(m, pair32_max(mloc) * sq);
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);  // m = -inf at the first block: 0
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      t[r] = __builtin_amdgcn_exp2f(fmaf(t[r], sq, -mnew));
      ps += t[r];
    }
    lsum = lsum * alpha + ps;
    m = mnew;
    // alpha is exactly 1 where the max did not move: skip the rescale when
    // that holds for the whole wave (bit-identical)
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int tt = 0; tt < 4; tt++) acc[tt] *= alpha;
    }
    // O^T += V^T . P^T on the bf16 MFMA (32x32x16), each product split as
    // V_hi.P_hi + V_hi.P_lo + V_lo.P_hi (x_hi = bf16(x), x_lo = bf16(x - x_hi):
    // ~2^-17 relative per product, fp32 accumulation; P is in [0, 1], so no
    // exponential amplifies it). Step s2 takes keys 16 s2 + 8(m/4) + 4h + m%4,
    // m = 0..7, exactly the lane's P registers t[8 s2 + m] and its two V^T
    // float4s at keys 16 s2 + 4h and 16 s2 + 8 + 4h.
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
      v8bf ph, pl;
#pragma unroll
      for (int m = 0; m < 8; m++) {
        const float x = t[8 * s2 + m];
        const __bf16 hb = (__bf16)x;
        ph[m] = hb;
        pl[m] = (__bf16)(x - (float)hb);
      }
#pragma unroll
      for (int tt = 0; tt < 4; tt++) {
        const int dq = 8 * s2 + 4 * h;  // dword of stored position 16 s2 + 8h
        const v8bf vh = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(&vth[b][32 * tt + j][dq]));
        const v8bf vl = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(&vtl[b][32 * tt + j][dq]));
        acc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, ph, acc[tt], 0, 0, 0);
        acc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, pl, acc[tt], 0, 0, 0);
        acc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vl, ph, acc[tt], 0, 0, 0);
      }
    }
    // K(kb+2) into the buffer K(kb) left before the last barrier; V(kb+1)
    // into the one V(kb-1) left. Kept after the P.V MFMAs: hoisted into the
    // softmax, the stash's work would wait there for this iteration's loads.
    __builtin_amdgcn_sched_barrier(0);
    stash_k(b, (int)((kb + 2) % 3));
    stash_v(b ^ 1);
    st = sn;
    __syncthreads();
  }
  // out[query][dim]: lane holds dims 32tt + 8(r/4) + 4h + r%4 of query j
  const float ltot = pair32_sum(lsum);
  const int64_t qi = q0 + j;
  if constexpr (SPLIT) {
    if (qi < Lq) {
      const int64_t row = (int64_t)blockIdx.y * Lq + qi;
      const int64_t sr = (int64_t)blockIdx.z * part.rows + row;
      float* dst = part.o + sr * part.heads * kHd + col;
#pragma unroll
      for (int tt = 0; tt < 4; tt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float4 o = {acc[tt][4 * g], acc[tt][4 * g + 1], acc[tt][4 * g + 2],
                            acc[tt][4 * g + 3]};
          *reinterpret_cast<float4*>(dst + 32 * tt + 8 * g + 4 * h) = o;
        }
      if (h == 0) part.ml[sr * part.heads + head] = float2{m, ltot};
    }
    return;
  }
  const float inv = 1.f / ltot;
  if (qi < Lq) {
    float* dst = O + qi * ldo + col;
#pragma unroll
    for (int tt = 0; tt < 4; tt++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 o = {acc[tt][4 * g] * inv, acc[tt][4 * g + 1] * inv, acc[tt][4 * g + 2] * inv,
                          acc[tt][4 * g + 3] * inv};
        *reinterpret_cast<float4*>(dst + 32 * tt + 8 * g + 4 * h) = o;
      }
  }
}

// out[row][head dims] = sum_s w_s o_s / sum_s w_s l_s, w_s = 2^(m_s - max m):
// the splits' partial softmax states combined. One thread per 4 dims.
__global__ void __launch_bounds__(256)
sdpa_merge_kernel(SdpaPart part, int splits, int64_t Lq, float* __restrict__ O, int64_t ldo) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = (int64_t)part.heads * (kHd / 4);
  if (idx >= part.rows * per_row) return;
  const int64_t row = idx / per_row;
  const int rem = (int)(idx - row * per_row);
  const int head = rem / (kHd / 4), d4 = rem - head * (kHd / 4);
  float mx = -INFINITY;
  for (int sp = 0; sp < splits; sp++)
    mx = fmaxf(mx, part.ml[((int64_t)sp * part.rows + row) * part.heads + head].x);
  float lt = 0.f;
  float4 o = {0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < splits; sp++) {
    const int64_t sr = (int64_t)sp * part.rows + row;
    const float2 ml = part.ml[sr * part.heads + head];
    const float w = __builtin_amdgcn_exp2f(ml.x - mx);  // an empty split: -inf - mx -> 0
    lt += w * ml.y;
    const float4 v = *reinterpret_cast<const float4*>(part.o + sr * part.heads * kHd +
                                                      (int64_t)head * kHd + 4 * d4);
    o.x += w * v.x;
    o.y += w * v.y;
    o.z += w * v.z;
    o.w += w * v.w;
  }
  const float inv = 1.f / lt;
  // rows of batch b's Lq queries are contiguous in O (row = b * Lq + q)
  *reinterpret_cast<float4*>(O + row * ldo + (int64_t)head * kHd + 4 * d4) =
      float4{o.x * inv, o.y * inv, o.z * inv, o.w * inv};
}

}  // namespace

// Waves per workgroup of a key-split launch: 8 (256 queries share each
// staged K / V block) from 512 queries up, else 2.
int sdpa_split_nw(int64_t Lq) { return Lq >= 512 ? 8 : 2; }

// Key splits for a sequence of Lq queries, Lk keys: the factor S that
// minimizes the rounds of resident workgroups per unit of work (rounds / S;
// the kernel's registers and LDS allow one 8-wave or two 2-wave workgroups
// per CU), each split keeping >= 3 key blocks and none empty; a split must
// beat the unsplit launch by 10% (the merge reads the partial outputs back).
// Depends on the sequence only, not on the batch, so stacked and separate
// calls give the same bits.
int sdpa_splits(int64_t Lq, int64_t Lk, int heads, int cu_count) {
  if (Lq >= 1024 || Lq <= 0 || Lk <= 0 || heads <= 0) return 1;  // many queries: no split
  if (const char* e = getenv("SDQ_SDPA_SPLIT")) {
    const int f = atoi(e);
    return f < 2 ? 1 : (f > 16 ? 16 : f);
  }
  const int64_t cus = cu_count > 0 ? cu_count : 256;
  const int nw = sdpa_split_nw(Lq);
  const int64_t groups = ceil_div(Lq, 32 * nw) * heads;
  const int64_t cap = nw == 8 ? cus : 2 * cus;
  // the unsplit launch (2-wave groups below 1024 queries)
  const double unsplit = (double)ceil_div(ceil_div(Lq, 64) * heads, 2 * cus);
  const int64_t nkb = ceil_div(Lk, kKB);
  const int64_t smax = nkb / 3 < 16 ? nkb / 3 : 16;
  int best = 1;
  double best_cost = unsplit;
  for (int64_t S = 2; S <= smax; S++) {
    if (ceil_div(nkb, ceil_div(nkb, S)) != S) continue;  // no empty split
    // rounds of resident groups, each walking 1/S of the keys (a group of
    // either width takes about as long per key block)
    const double cost = (double)ceil_div(groups * S, cap) / (double)S;
    if (cost < best_cost) {
      best_cost = cost;
      best = (int)S;
    }
  }
  return best_cost <= 0.9 * unsplit ? best : 1;
}

int64_t sdpa_part_floats(int64_t Lq, int64_t Lk, int heads, int batch, int cu_count) {
  const int S = sdpa_splits(Lq, Lk, heads, cu_count);
  if (S <= 1) return 0;
  const int64_t rows = (int64_t)batch * Lq;
  return (int64_t)S * rows * heads * (kHd + 2);
}

hipError_t launch_sdpa(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                       int64_t ldv, float* out, int64_t ldo, int64_t Lq, int64_t Lk, int heads,
                       hipStream_t s, int batch, float* part, int cu_count) {
  if (Lq <= 0 || batch == 0) return hipSuccess;
  if (Lk <= 0 || heads <= 0 || batch < 0 || batch > 65535) return hipErrorInvalidValue;
  const float scale_log2e = (1.f / sqrtf((float)kHd)) * 1.4426950408889634f;
  // waves per workgroup (32 queries each); SDQ_SDPA_NW = 2, 4 or 8 overrides
  static const int forced = [] {
    const char* e = getenv("SDQ_SDPA_NW");
    const int v = e ? atoi(e) : 0;
    return v == 2 || v == 4 || v == 8 ? v : 0;
  }();
  const int nw = forced ? forced : Lq >= 1024 ? 8 : 2;
  const int S = part && !forced ? sdpa_splits(Lq, Lk, heads, cu_count) : 1;
  if (S > 1) {
    // key splits, then the merge (part: sdpa_part_floats floats)
    SdpaPart pp{part, nullptr, (int64_t)batch * Lq, heads, 0};
    pp.ml = reinterpret_cast<float2*>(part + (int64_t)S * pp.rows * heads * kHd);
    pp.kbs = (int)ceil_div(ceil_div(Lk, kKB), S);
    const int snw = sdpa_split_nw(Lq);
    const int qgroups = (int)ceil_div(Lq, 32 * snw);
    const dim3 grid((unsigned)(qgroups * heads), (unsigned)batch, (unsigned)S);
    if (snw == 8)
      hipLaunchKernelGGL((sdpa_kernel<8, true>), grid, dim3(512), 0, s, q, ldq, k, ldk, v, ldv,
                         out, ldo, Lq, Lk, qgroups, scale_log2e, pp);
    else
      hipLaunchKernelGGL((sdpa_kernel<2, true>), grid, dim3(128), 0, s, q, ldq, k, ldk, v, ldv,
                         out, ldo, Lq, Lk, qgroups, scale_log2e, pp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t n = pp.rows * heads * (kHd / 4);
    hipLaunchKernelGGL(sdpa_merge_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, pp,
                       S, Lq, out, ldo);
    return hipGetLastError();
  }
  auto go = [&](auto nwc) {
    constexpr int NW = decltype(nwc)::value;
    const int qgroups = (int)ceil_div(Lq, 32 * NW);
    hipLaunchKernelGGL((sdpa_kernel<NW, false>), dim3((unsigned)(qgroups * heads), (unsigned)batch),
                       dim3(NW * 64), 0, s, q, ldq, k, ldk, v, ldv, out, ldo, Lq, Lk, qgroups,
                       scale_log2e, SdpaPart{});
  };
  if (nw == 8)
    go(std::integral_constant<int, 8>{});
  else if (nw == 4)
    go(std::integral_constant<int, 4>{});
  else
    go(std::integral_constant<int, 2>{});
  return hipGetLastError();
}

}  // namespace sdq
