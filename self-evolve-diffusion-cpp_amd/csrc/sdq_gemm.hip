// int8 x int8 -> int32 MFMA GEMM with the fused fp32 epilogue (gfx950).
//
// Computes, for every output (i = activation row m, j = weight row n):
//   acc = sum_k aq[m,k] * wq[n,k]                 src/core/qgemm.cpp:107-138
//   y   = fl(fl((float)acc) * fl(as[m] * bs[n]))  src/core/qgemm.cpp:123-124,135
//   y   = fl(y + bias[n])                         src/model/ovi_dit.cpp:71-79
//   then GELU / gated fma residual / plain residual (ovi_dit.cpp:132-159).
// Integer accumulation is exact and order-free, and every fp32 step is one
// correctly rounded IEEE operation (contraction is off in this file), so the
// result is bit-identical to the reference CPU path.
//
// MFMA roles: the WEIGHT fragment is the instruction's A operand (rows = n)
// and the ACTIVATION fragment its B operand (columns = m), so the 32x32 i32
// result C^T[n][m] of v_mfma_i32_32x32x32_i8 lands as groups of 4
// consecutive n of one m per lane: lane l, accumulator register r holds
// m = l & 31, n = 8(r >> 2) + 4(l >> 5) + (r & 3), i.e. four 16-byte
// row-contiguous stores of Y[m, n..n+3] per 32x32 block. The persistent
// kernels read the same fragments as v_mfma_i32_16x16x64_i8 operands (same
// roles; their result layout is described at qgemm_persist).
#include "sdq_internal.h"
#include "sdq_device.h"

#include <cstdlib>
#include <type_traits>

#pragma clang fp contract(off)

// Row tiles per group of the persistent kernels' XCD-aware tile order (a
// group's tiles share A panels in the XCD's L2).
#ifndef SDQ_PERSIST_GROUP_M
#define SDQ_PERSIST_GROUP_M 4
#endif

namespace sdq {

namespace {

using namespace dev;

__device__ __forceinline__ void load4(const float* __restrict__ p, int64_t n0, int64_t N, bool vec,
                                      float v[4]) {
  if (vec) {
    const float4 x = *reinterpret_cast<const float4*>(p + n0);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  } else {
#pragma unroll
    for (int r = 0; r < 4; r++) v[r] = (n0 + r < N) ? p[n0 + r] : 0.f;
  }
}

// Epilogue for the accumulators of Y[m, n0..n0+3] held by one lane.
__device__ __forceinline__ void store_out(const int acc[4], int64_t m, int64_t n0, int64_t M,
                                          int64_t N, float as_m, const float* __restrict__ bs,
                                          const EpiArgs& e, void* Y, bool vec) {
  if (m >= M || n0 >= N) return;
  const int64_t o = m * N + n0;
  if (e.kind == SDQ_EPI_ACC) {
    int* y = static_cast<int*>(Y) + o;
    if (vec) {
      *reinterpret_cast<int4*>(y) = make_int4(acc[0], acc[1], acc[2], acc[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; r++)
        if (n0 + r < N) y[r] = acc[r];
    }
    return;
  }
  // bs is padded to a multiple of 256 entries and 16-byte aligned.
  const float4 s4 = *reinterpret_cast<const float4*>(bs + n0);
  const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
  float v[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const float s = as_m * sv[r];
    const float a = (float)acc[r];
    v[r] = e.kzero ? 0.f : a * s;
  }
  if (e.bias) {
    float b[4];
    load4(e.bias, n0, N, vec, b);
#pragma unroll
    for (int r = 0; r < 4; r++) v[r] = v[r] + b[r];
  }
  if (e.kind == SDQ_EPI_GELU) {
#pragma unroll
    for (int r = 0; r < 4; r++) v[r] = gelu_tanh(v[r]);
  } else if (e.kind == SDQ_EPI_GATED) {
    float g[4], x[4];
    load4(e.gate, n0, N, vec, g);
    load4(e.resid + m * N, n0, N, vec, x);
    if (e.gate_fma) {
#pragma unroll
      for (int r = 0; r < 4; r++) v[r] = __builtin_fmaf(v[r], g[r], x[r]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float p = v[r] * g[r];
        v[r] = x[r] + p;
      }
    }
  } else if (e.kind == SDQ_EPI_RESID) {
    float x[4];
    load4(e.resid + m * N, n0, N, vec, x);
#pragma unroll
    for (int r = 0; r < 4; r++) v[r] = x[r] + v[r];
  }
  float* y = static_cast<float*>(Y) + o;
  if (vec) {
    *reinterpret_cast<float4*>(y) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int r = 0; r < 4; r++)
      if (n0 + r < N) y[r] = v[r];
  }
}

// Stores one 32x32 accumulator block: n_lane = n of this lane's group 0.
__device__ __forceinline__ void store_block(const v16i& acc, int64_t m, int64_t n_lane, int64_t M,
                                            int64_t N, float as_m, const float* __restrict__ bs,
                                            const EpiArgs& e, void* Y, bool vec) {
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int a4[4] = {acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
    store_out(a4, m, n_lane + 8 * g, M, N, as_m, bs, e, Y, vec);
  }
}

// Epilogue of Y[m, n0..n0+3] with the per-column operands already in
// registers (weight scale s4, bias b4, gate g4); only the residual, when the
// epilogue has one, is read from global memory here.
__device__ __forceinline__ void finish4(const int* acc, int64_t m, int64_t n0, int64_t M, int64_t N,
                                        float as_m, const float4 s4, const float4 b4,
                                        const float4 g4, const EpiArgs& e, void* Y, bool vec) {
  if (m >= M || n0 >= N) return;
  const int64_t o = m * N + n0;
  if (e.kind == SDQ_EPI_ACC) {
    int* y = static_cast<int*>(Y) + o;
    if (vec) {
      *reinterpret_cast<int4*>(y) = make_int4(acc[0], acc[1], acc[2], acc[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; r++)
        if (n0 + r < N) y[r] = acc[r];
    }
    return;
  }
  const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
  const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
  const float gv[4] = {g4.x, g4.y, g4.z, g4.w};
  float v[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const float s = as_m * sv[r];
    const float a = (float)acc[r];
    v[r] = e.kzero ? 0.f : a * s;
  }
  if (e.bias) {
#pragma unroll
    for (int r = 0; r < 4; r++) v[r] = v[r] + bv[r];
  }
  if (e.kind == SDQ_EPI_GELU) {
#pragma unroll
    for (int r = 0; r < 4; r++) v[r] = gelu_tanh(v[r]);
  } else if (e.kind == SDQ_EPI_GATED || e.kind == SDQ_EPI_RESID) {
    float x[4];
    load4(e.resid + m * N, n0, N, vec, x);
    if (e.kind == SDQ_EPI_RESID) {
#pragma unroll
      for (int r = 0; r < 4; r++) v[r] = x[r] + v[r];
    } else if (e.gate_fma) {
#pragma unroll
      for (int r = 0; r < 4; r++) v[r] = __builtin_fmaf(v[r], gv[r], x[r]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float p = v[r] * gv[r];
        v[r] = x[r] + p;
      }
    }
  }
  float* y = static_cast<float*>(Y) + o;
  if (vec) {
    *reinterpret_cast<float4*>(y) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int r = 0; r < 4; r++)
      if (n0 + r < N) y[r] = v[r];
  }
}

// ---------------------------------------------------------------------------
// Tiled kernel: one workgroup computes a BN (weight rows) x BM (activation
// rows) output tile. Each pipeline stage moves KS k-fragments (32 bytes of K
// each) of both panels global -> LDS with direct-to-LDS 16-byte loads (no
// VGPR staging) into a ring of STAGES buffers; STAGES-1 stages are in
// flight while one is consumed, and each wave waits only for its own oldest
// stage (vmcnt) before the workgroup barrier. WN x WM waves each own
// FN x FM 32x32 accumulator blocks.
template <int BN, int BM, int WN, int WM, int KS, int STAGES>
__global__ void __launch_bounds__(WN* WM * 64, 1)
qgemm_tiled(const int8_t* __restrict__ wt, const float* __restrict__ bs,
            const int8_t* __restrict__ at, const float* __restrict__ as, int64_t M, int64_t N,
            int64_t KFp, int tiles_n, int tiles_m, EpiArgs epi, void* Y, int vec) {
  constexpr int NW = WN * WM;
  constexpr int RBN = BN / 32, RBM = BM / 32;
  constexpr int FN = RBN / WN, FM = RBM / WM;
  constexpr int WFR = RBN * KS, AFR = RBM * KS, SFR = WFR + AFR;
  constexpr int WLD = WFR / NW, ALD = AFR / NW, LPW = WLD + ALD;
  constexpr int STAGE = SFR * 1024;
  static_assert(WFR % NW == 0 && AFR % NW == 0, "stage fragments must split evenly over waves");
  static_assert(NW % KS == 0, "waves must be a multiple of k-fragments per stage");
  static_assert(STAGES >= 2 && (STAGES - 1) * LPW < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char lds[STAGES * STAGE];

  const int lane = threadIdx.x & 63;
  // Wave index as a scalar: keeps every per-wave offset in SGPRs.
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = w % WN, wm = w / WN;

  // ---- tile order: spread over the 8 XCDs (workgroup b runs on XCD b % 8),
  // each XCD gets a contiguous run of the grouped tile order so the tiles
  // resident on one XCD share activation and weight panels in its L2.
  const int T = tiles_n * tiles_m;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, jx = bid >> 3, q8 = T >> 3, r8 = T & 7;
  const int lin = xcd * q8 + (xcd < r8 ? xcd : r8) + jx;
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * tiles_n;
  const int g = lin / per_group;
  const int first_m = g * GROUP_M;
  const int gsz = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  const int rem = lin - g * per_group;
  const int tm = first_m + rem % gsz;
  const int tn = rem / gsz;

  // ---- per-column epilogue operands of this tile (weight scale, bias,
  // gate) staged in LDS and per-row activation scales in registers, so the
  // epilogue does not wait on global loads. Visible to all waves after the
  // first pipeline barrier.
  __shared__ __attribute__((aligned(16))) float col_ops[3][BN];
  for (int t = threadIdx.x; t < BN; t += NW * 64) {
    const int64_t n = (int64_t)tn * BN + t;  // < Np: bs is zero padded
    col_ops[0][t] = bs[n];
    col_ops[1][t] = (epi.bias && n < N) ? epi.bias[n] : 0.f;
    col_ops[2][t] = (epi.gate && n < N) ? epi.gate[n] : 0.f;
  }
  float as_reg[FM];
#pragma unroll
  for (int j = 0; j < FM; j++) {
    const int64_t m = (int64_t)tm * BM + (wm * FM + j) * 32 + (lane & 31);
    as_reg[j] = (m < M) ? as[m] : 0.f;
  }

  // ---- per-wave global offsets (stage 0). Stage fragment f = t*NW + w,
  // weight fragments first; with NW % KS == 0 all of a wave's fragments sit
  // at k index w % KS and the row block advances by NW/KS per t.
  const uint32_t lane_off = (uint32_t)lane * 16u;
  const int64_t wbase = ((int64_t)(tn * RBN + w / KS) * KFp + (w % KS)) * 1024;
  const int64_t abase = ((int64_t)(tm * RBM + w / KS) * KFp + (w % KS)) * 1024;
  const int64_t tstride = (int64_t)(NW / KS) * KFp * 1024;

  v16i acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; i++)
#pragma unroll
    for (int j = 0; j < FM; j++) acc[i][j] = v16i{};

  const int nks = (int)(KFp / KS);

  auto issue = [&](int ks) {
    char* buf = lds + (ks % STAGES) * STAGE;
    const int64_t koff = (int64_t)ks * KS * 1024;
#pragma unroll
    for (int t = 0; t < WLD; t++) {
      const int8_t* src = wt + (wbase + koff + t * tstride);
      __builtin_amdgcn_global_load_lds(src + lane_off, buf + (t * NW + w) * 1024, 16, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < ALD; t++) {
      const int8_t* src = at + (abase + koff + t * tstride);
      __builtin_amdgcn_global_load_lds(src + lane_off, buf + WFR * 1024 + (t * NW + w) * 1024, 16,
                                       0, 0);
    }
  };
  // Operand fragments of one stage, double buffered in registers.
  struct Frags {
    v4i a[KS][FN], b[KS][FM];
  };
  auto lds_read = [&](int ks, Frags& f) {
    const char* cb = lds + (ks % STAGES) * STAGE;
#pragma unroll
    for (int kk = 0; kk < KS; kk++) {
#pragma unroll
      for (int i = 0; i < FN; i++)
        f.a[kk][i] = *reinterpret_cast<const v4i*>(cb + ((wn * FN + i) * KS + kk) * 1024 + lane_off);
#pragma unroll
      for (int j = 0; j < FM; j++)
        f.b[kk][j] = *reinterpret_cast<const v4i*>(cb + WFR * 1024 +
                                                   ((wm * FM + j) * KS + kk) * 1024 + lane_off);
    }
  };
  auto mma = [&](const Frags& f, int kk) {
#pragma unroll
    for (int i = 0; i < FN; i++)
#pragma unroll
      for (int j = 0; j < FM; j++)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[kk][i], f.b[kk][j], acc[i][j], 0, 0, 0);
  };
  // Waits until this wave's loads of stage `next` have landed (later stages
  // may stay in flight), then syncs the workgroup.
  auto wait_and_sync = [&](int next) {
    if (next + STAGES - 2 < nks)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 2) * LPW));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    asm volatile("s_barrier" ::: "memory");
  };
  // One pipeline step: MFMAs of stage ks from `cur` (first k-fragment, then
  // the rest), with the barrier for stage ks+1, the refill of the buffer
  // that stage ks occupied, and the LDS reads of stage ks+1 into `nxt`
  // placed between them so the MFMA pipe stays busy across the barrier and
  // the LDS latency.
  auto step = [&](int ks, const Frags& cur, Frags& nxt) {
    mma(cur, 0);
    if (ks + 1 < nks) {
      wait_and_sync(ks + 1);
      if (ks + STAGES < nks) issue(ks + STAGES);
      lds_read(ks + 1, nxt);
    }
#pragma unroll
    for (int kk = 1; kk < KS; kk++) mma(cur, kk);
  };

#pragma unroll
  for (int s0 = 0; s0 < STAGES; s0++)
    if (s0 < nks) issue(s0);
  if (STAGES - 1 < nks)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 1) * LPW));
  else
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  asm volatile("s_barrier" ::: "memory");
  Frags f0, f1;
  lds_read(0, f0);
  int ks = 0;
  for (; ks + 1 < nks; ks += 2) {
    step(ks, f0, f1);
    step(ks + 1, f1, f0);
  }
  if (ks < nks) step(ks, f0, f1);

  // ---- epilogue
  const int64_t mb = (int64_t)tm * BM + wm * FM * 32 + (lane & 31);
  const int nl0 = wn * FN * 32 + (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < FN; i++) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int nl = nl0 + i * 32 + 8 * g;
      const float4 s4 = *reinterpret_cast<const float4*>(&col_ops[0][nl]);
      const float4 b4 = *reinterpret_cast<const float4*>(&col_ops[1][nl]);
      const float4 g4 = *reinterpret_cast<const float4*>(&col_ops[2][nl]);
      const int64_t n0 = (int64_t)tn * BN + nl;
#pragma unroll
      for (int j = 0; j < FM; j++) {
        const int a4[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                           acc[i][j][4 * g + 3]};
        finish4(a4, mb + j * 32, n0, M, N, as_reg[j], s4, b4, g4, epi, Y, vec);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent tiled kernel (the main path; needs 16-byte vector epilogue
// access). gridDim.x workgroups walk the tile list with stride gridDim.x,
// and the LDS pipeline runs straight across tile boundaries: the next
// tile's first stages are prefetched while the current tile's last stages
// compute, so the epilogue of one tile overlaps the loads of the next.
//
// A pipeline stage holds two k-fragments (64 bytes of K) of the tile's
// weight and activation panels: one k-step of v_mfma_i32_16x16x64_i8,
// whose operands are read straight out of the fragment layout (the lane
// mapping is at `off16` below). Each step (one stage) runs in two halves:
//   half 0: the MFMAs of the wave's first half of weight rows against all
//           its activation columns, interleaved with the LDS reads of the
//           second half's weight operands;
//   wait until this wave's loads of the next stage have landed, barrier;
//   half 1: the MFMAs of the second half of weight rows, interleaved with
//           the LDS-DMA of the stage STAGES ahead (into the buffer this
//           stage used) and the LDS reads of the next stage's first-half
//           weight operands and activation operands.
// The 16x16x64 form moves the same LDS bytes and holds the same
// accumulator registers per k as 32x32x32 tiles of the same wave tile, at
// less power per operation: under the power limit the clock runs ~18%
// higher (1.67 vs 1.41 GHz on the north star).
// The steady state is branch-free: past the last stage the issue cursor
// uses zero-range buffer descriptors, so its loads fetch nothing and land
// in a buffer no remaining stage reads, and every wait keeps the same
// count. On this GPU family one counter (vmcnt) tracks loads and stores;
// a wait counts younger loads only, so pending epilogue stores can only
// make a wait longer. Per-tile weight scales, bias, gate and activation
// scales arrive by LDS-DMA into a double buffer after the tile's first
// stage.
// SPLITK: the work items are (tile, k-range) pairs, `splits` contiguous
// k-ranges per tile, each writing raw int32 sums to its own [M,N] slice of
// Y (EPI_ACC); splitk_reduce adds the slices and applies the epilogue.
// The grouped launches' problem table (GROUPED), or nothing.
struct NoGroup {};
template <bool GROUPED>
using GroupArg = typename std::conditional<GROUPED, GemmGroup, NoGroup>::type;
// Field reads that compile for both argument types (only called when GROUPED).
__device__ __forceinline__ int group_total(const GemmGroup& g) { return g.total; }
__device__ __forceinline__ int group_total(const NoGroup&) { return 0; }
__device__ __forceinline__ int64_t group_m(const GemmGroup& g, int p) { return g.p[p].M; }
__device__ __forceinline__ int64_t group_m(const NoGroup&, int) { return 0; }
__device__ __forceinline__ int64_t group_n(const GemmGroup& g, int p) { return g.p[p].N; }
__device__ __forceinline__ int64_t group_n(const NoGroup&, int) { return 0; }
__device__ __forceinline__ void* group_y(const GemmGroup& g, int p) { return g.p[p].Y; }
__device__ __forceinline__ void* group_y(const NoGroup&, int) { return nullptr; }
__device__ __forceinline__ const float* group_resid(const GemmGroup& g, int p) {
  return g.p[p].resid;
}
__device__ __forceinline__ const float* group_resid(const NoGroup&, int) { return nullptr; }
__device__ __forceinline__ int group_kind(const GemmGroup& g, int p) { return g.p[p].kind; }
__device__ __forceinline__ int group_kind(const NoGroup&, int) { return 0; }
__device__ __forceinline__ bool group_fma(const GemmGroup& g, int p) { return g.p[p].gate_fma != 0; }
__device__ __forceinline__ bool group_fma(const NoGroup&, int) { return true; }
__device__ __forceinline__ bool group_bias(const GemmGroup& g, int p) { return g.p[p].bias != nullptr; }
__device__ __forceinline__ bool group_bias(const NoGroup&, int) { return false; }

template <int BN, int BM, int WN, int WM, int KS, int STAGES, int OCC, int EPI, bool BIAS,
          bool SPLITK, bool GROUPED = false>
__global__ void __launch_bounds__(WN* WM * 64, OCC)
qgemm_persist(const int8_t* __restrict__ wt, ColOps cols, const int8_t* __restrict__ at,
              const float* __restrict__ as, int64_t M, int64_t N, int64_t KFp, int tiles_n,
              int tiles_m, EpiArgs epi, void* Y, int splits, GroupArg<GROUPED> grp) {
  static_assert(!SPLITK || EPI == SDQ_EPI_ACC, "split-K partials are raw accumulators");
  static_assert(!(GROUPED && SPLITK), "grouped launches do not split K");
  static_assert(EPI != kEpiMixed || (GROUPED && !BIAS), "mixed epilogues come from a group's table");
  static_assert(KS == 2, "a 16x16x64 k-step spans the two k-fragments of a stage");
  constexpr int NW = WN * WM;
  constexpr int RBN = BN / 32, RBM = BM / 32;
  constexpr int FN = RBN / WN, FM = RBM / WM;
  constexpr int WFR = RBN * KS, AFR = RBM * KS, SFR = WFR + AFR;
  constexpr int WLD = WFR / NW, ALD = AFR / NW, LPW = WLD + ALD;
  constexpr int STAGE = SFR * 1024;
  static_assert(WFR % NW == 0 && AFR % NW == 0, "stage fragments must split evenly over waves");
  static_assert(NW % KS == 0, "waves must be a multiple of k-fragments per stage");
  static_assert(NW >= 4, "four waves load the per-tile operands");
  static_assert(STAGES >= 2 && (STAGES - 1) * LPW < 64, "vmcnt range");
  static_assert(LPW <= 2 * FN * FM && FN <= 2 * FN * FM, "memory slots per MFMA");
  static_assert(BN <= 256 && BM <= 256, "one 1 KB DMA per per-tile operand");
  // GELU's epilogue spills SGPRs, and the grouped kernels read their
  // problem table into spilled SGPRs; the reloads can sit next to a DMA
  constexpr int kDmaNop = (EPI == SDQ_EPI_GELU || GROUPED) ? 4 : 0;
  __shared__ __attribute__((aligned(1024))) char lds[STAGES * STAGE];
  __shared__ __attribute__((aligned(16))) float colb[2][3][BN];
  __shared__ __attribute__((aligned(16))) float rowb[2][BM];
  // Epilogue transpose scratch of each wave, beside the operand ring: 4 KB
  // (a whole 32x32 block) when LDS has room, else 2 KB (the block in two
  // halves of 16 rows). Both persistent configurations take 2 KB: 256x256
  // 128 + 8 + 16 KB, 128x128 twice 64 + 4 + 8 KB. Owning it keeps the ring
  // refilling through the tile's last stage (borrowing a stage buffer would
  // hold that refill until after the epilogue: 1% slower at 27280 rows).
  constexpr int kLdsPipe = STAGES * STAGE + (2 * 3 * BN + 2 * BM) * 4;
  constexpr bool kFullScr = OCC * (kLdsPipe + NW * 4096) <= 160 * 1024;
  static_assert(kFullScr || OCC * (kLdsPipe + NW * 2048) <= 160 * 1024,
                "LDS: operand ring plus transpose scratch");
  constexpr int kScrBytes = kFullScr ? 4096 : 2048;
  constexpr int kHalves = kFullScr ? 1 : 2;
  __shared__ __attribute__((aligned(1024))) char escr[NW * kScrBytes];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = w % WN, wm = w / WN;
  const uint32_t lane_off = (uint32_t)lane * 16u;

  const int T = GROUPED ? group_total(grp) : tiles_n * tiles_m;
  const int S = SPLITK ? splits : 1;
  const int TS = T * S;  // work items
  const int G = gridDim.x;
  const int ntile = (TS - (int)blockIdx.x + G - 1) / G;
  const int klen = (int)(KFp / S);  // k-fragments per work item
  const int nks = klen / KS;

  // Work item i of this workgroup -> (tm, tn, k-range ks) of problem pb:
  // XCD-aware grouped order applied to the virtual block id blockIdx.x + i*G
  // (G is a multiple of 8, so it stays on this XCD); a grouped launch first
  // finds the problem whose tiles hold the item.
  auto coords = [&](int i, int& tm, int& tn, int& ks, int& pb) {
    const int bid = (int)blockIdx.x + i * G;
    const int xcd = bid & 7, jx = bid >> 3, q8 = TS >> 3, r8 = TS & 7;
    int lin = xcd * q8 + (xcd < r8 ? xcd : r8) + jx;
    ks = 0;
    if constexpr (SPLITK) {
      ks = lin / T;
      lin -= ks * T;
    }
    constexpr int GROUP_M = SDQ_PERSIST_GROUP_M;
    pb = 0;
    if constexpr (GROUPED) {
#pragma unroll
      for (int q = 1; q < kMaxGemmGroup; q++)
        if (q < grp.count && lin >= grp.p[q].tile0) pb = q;
      pb = __builtin_amdgcn_readfirstlane(pb);  // uniform: the table reads stay scalar
      lin -= grp.p[pb].tile0;
      const int ptn = grp.p[pb].tiles_n, ptm = grp.p[pb].tiles_m;
      const int per_group = GROUP_M * ptn;
      const int g = lin / per_group;
      const int first_m = g * GROUP_M;
      const int gsz = (ptm - first_m) < GROUP_M ? (ptm - first_m) : GROUP_M;
      const int rem = lin - g * per_group;
      tm = first_m + rem % gsz;
      tn = rem / gsz;
    } else {
      const int per_group = GROUP_M * tiles_n;
      const int g = lin / per_group;
      const int first_m = g * GROUP_M;
      const int gsz = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
      const int rem = lin - g * per_group;
      tm = first_m + rem % gsz;
      tn = rem / gsz;
    }
  };

  // ---- issue cursor: the next stage to load (segment cj, stage cks), with
  // buffer descriptors over that tile's weight / activation panels (raw
  // buffers: out-of-range reads return 0) so every load is one SGPR
  // descriptor + SGPR offset + the lane's 16-byte VGPR offset. Past the
  // last segment the descriptors have zero range.
  constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, valid
  const int wpanel = RBN * (int)KFp * 1024, apanel = RBM * (int)KFp * 1024;
  const int wso0 = ((w / KS) * (int)KFp + (w % KS)) * 1024;
  const int tso = (NW / KS) * (int)KFp * 1024;
  const uint32_t lds0 = lds_addr32(lds) + (uint32_t)w * 1024u;
  int cj = 0, cks = 0, ctm = 0, ctn = 0, cgs = 0, csp = 0, cpb = 0;
  int wso = wso0;
  bool col_due = true;  // the segment's first stage was issued; its column loads follow
  v4u wr, ar;
  auto set_tile = [&](int i) {
    coords(i, ctm, ctn, csp, cpb);
    if constexpr (GROUPED) {
      wr = raw_rsrc(grp.p[cpb].wt + (int64_t)ctn * wpanel, (uint32_t)wpanel);
      ar = raw_rsrc(grp.p[cpb].at + (int64_t)ctm * apanel, (uint32_t)apanel);
    } else {
      wr = raw_rsrc(wt + (int64_t)ctn * wpanel, (uint32_t)wpanel);
      ar = raw_rsrc(at + (int64_t)ctm * apanel, (uint32_t)apanel);
    }
    wso = wso0 + csp * klen * 1024;  // the work item's first k-fragment
  };
  set_tile(0);
  // Load t (0..LPW-1) of the cursor's stage: WLD weight, then ALD
  // activation fragments, 1 KB each.
  auto dma_stage = [&](int t) {
    const uint32_t buf = lds0 + (uint32_t)(((unsigned)cgs % STAGES) * STAGE);
    if (t < WLD)
      dma16<kDmaNop>(wr, lane_off, (uint32_t)(wso + t * tso), buf + (uint32_t)(t * NW * 1024));
    else
      dma16<kDmaNop>(ar, lane_off, (uint32_t)(wso + (t - WLD) * tso),
            buf + (uint32_t)((WFR + (t - WLD) * NW) * 1024));
  };
  auto dma_row = [&](const float* src, int64_t off, int count, const float* dst) {
    if (lane * 4 < count)
      dma16<kDmaNop>(raw_rsrc(src + off, (uint32_t)count * 4u), lane_off, 0u, lds_addr32(dst));
  };
  // After a stage's loads: the per-tile column operands (once per segment,
  // younger than the segment's first stage), then the cursor moves on.
  auto advance = [&]() {
    if (col_due) {
      col_due = false;
      const int par = cj & 1;
      if constexpr (GROUPED) {
        const GemmProblem& q = grp.p[cpb];
        if (w < 3) {
          const float* src = w == 0 ? q.scale : (w == 1 ? q.bias : q.gate);
          if (src) dma_row(src, (int64_t)ctn * BN, BN, &colb[par][w][0]);
        } else if (w == 3) {
          dma_row(q.as, (int64_t)ctm * BM, BM, &rowb[par][0]);
        }
      } else {
        if (w < 3) {
          const float* src = w == 0 ? cols.scale : (w == 1 ? cols.bias : cols.gate);
          if (src) dma_row(src, (int64_t)ctn * BN, BN, &colb[par][w][0]);
        } else if (w == 3) {
          dma_row(as, (int64_t)ctm * BM, BM, &rowb[par][0]);
        }
      }
    }
    cgs++;
    wso += KS * 1024;
    if (++cks == nks) {
      if (++cj < ntile) {
        cks = 0;
        set_tile(cj);
        col_due = true;
      } else {
        wr = raw_rsrc(wt, 0u);
        ar = raw_rsrc(at, 0u);
      }
    }
  };

  // The stages' LDS image read as v_mfma_i32_16x16x64_i8 operands. Such an
  // operand holds 16 rows (lane l: row l & 15) and 64 k-bytes, spread over
  // the lanes the same way for both operands, so one 16-byte read per lane
  // from the stage's two k-fragments of a 32-row block serves as one: lane
  // l takes k-fragment l >> 5, fragment lane (l & 15) + 32((l >> 4) & 1),
  // plus 16 rows for the block's second half. Per stage: XN weight operands
  // (x: 16 rows), YM activation operands (y: 16 columns), XN x YM
  // accumulators of 4 registers (result lane l, register r: n = 16x +
  // 4(l >> 4) + r, m = 16y + (l & 15)).
  constexpr int XN = 2 * FN, YM = 2 * FM;
  const uint32_t off16 = (uint32_t)(lane >> 5) * 1024u +
                         (uint32_t)((lane & 15) + 32 * ((lane >> 4) & 1)) * 16u;
  struct Ops16 {
    v4i a[XN], b[YM];
  };
  Ops16 o16;
  v4i acc16[XN][YM];
  // Operand f of the stage in buffer cb: weight operands 0..XN-1, then
  // activation operands.
  auto read16 = [&](const char* cb, int f) {
    if (f < XN)
      o16.a[f] = *reinterpret_cast<const v4i*>(cb + (wn * FN + (f >> 1)) * KS * 1024 + off16 +
                                               (f & 1) * 256);
    else
      o16.b[f - XN] = *reinterpret_cast<const v4i*>(
          cb + WFR * 1024 + (wm * FM + ((f - XN) >> 1)) * KS * 1024 + off16 + ((f - XN) & 1) * 256);
  };
  // A tile's first stage starts from zero (no separate clearing pass).
  auto mma16 = [&](int x, int y, bool first) {
    acc16[x][y] = __builtin_amdgcn_mfma_i32_16x16x64_i8(o16.a[x], o16.b[y],
                                                        first ? v4i{} : acc16[x][y], 0, 0, 0);
  };
  // One pipeline step (stage gs) in two halves:
  //   half 0: weight operands 0..FN-1 against every activation operand,
  //           interleaved with the LDS reads of weight operands FN..XN-1;
  //   wait until this wave's loads of the next stage landed and every
  //   wave read buffer gs (vmcnt, lgkmcnt 0, barrier);
  //   half 1: weight operands FN..XN-1, activation-operand major (each
  //           activation register is free after its last use), interleaved
  //           with the LDS-DMA of the stage STAGES ahead into buffer gs and
  //           the reads of the next stage's weight operands 0..FN-1 and
  //           activation operands.
  auto step16 = [&](int gs, auto first_tag) {
    constexpr bool First = decltype(first_tag)::value;
    const char* cb = lds + ((unsigned)gs % STAGES) * STAGE;
#pragma unroll
    for (int i = 0; i < FN * YM; i++) {
      mma16(i / YM, i % YM, First);
      if (i < FN) read16(cb, FN + i);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 2) * LPW) & ~(15 << 8));
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const char* nb = lds + ((unsigned)(gs + 1) % STAGES) * STAGE;
#pragma unroll
    for (int i = 0; i < FN * YM; i++) {
      mma16(FN + i % FN, i / FN, First);
      if (i < LPW) dma_stage(i);
      if (i < FN) read16(nb, i);
      if (i % FN == FN - 1) read16(nb, XN + i / FN);
      __builtin_amdgcn_sched_barrier(0);
    }
    advance();
  };
  const std::true_type first_stage;
  const std::false_type next_stage;

  // prologue: STAGES stages in flight, stage 0 landed
#pragma unroll
  for (int s = 0; s < STAGES; s++) {
#pragma unroll
    for (int t = 0; t < LPW; t++) dma_stage(t);
    advance();
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm((STAGES - 1) * LPW));
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int f = 0; f < FN; f++) read16(lds, f);
#pragma unroll
  for (int f = 0; f < YM; f++) read16(lds, XN + f);

  // Epilogue memory goes through buffer descriptors too: masked lanes
  // (outside M x N) get an offset beyond the descriptor's range, which the
  // hardware drops on stores and reads as zero on loads.
  constexpr int kOutOfRange = (int)0x80000000u;
  constexpr int kBigRange = 0x7FFFFFF0;
  // Output rows are written once, in whole 128-byte segments: streaming
  // (non-temporal) stores keep them from displacing the operand panels in L2.
  constexpr int kStreamStore = 2;
  // Epilogue lane roles. Each 32x32 output block goes through LDS: from
  // the MFMA layout (four 16x16 quarters) to the row layout, where a lane
  // holds rows rr + 8i (i = 0..3), chunk rc, so eight consecutive lanes
  // store one 128-byte row segment.
  const int rr = lane >> 3, rc = lane & 7;
  const int ldy4 = (int)N * 4;
  const int wrow = wm * FM * 32, wcol = wn * FN * 32;  // this wave's block in the tile
  const int voff_lane = (wrow + rr) * ldy4 + (wcol + 4 * rc) * 4;
  int gs = 0;
  for (int j = 0; j < ntile; j++) {
    const int nst = nks;  // >= STAGES
    step16(gs++, first_stage);
    for (int q = 1; q < nst; q++) step16(gs++, next_stage);
    // Transpose scratch of this wave: 1 KB slots, slot t holding block rows
    // 8t..8t+7 (8t+7 mod 16 with 2 KB; 128 bytes each, 16-byte chunks
    // XOR-swizzled by the row so both access patterns are bank-conflict
    // free).
    char* const scr = escr + w * kScrBytes;
    constexpr int kSlot = 1024;
    // ---- epilogue of tile j
    int tm, tn, ksp, pb;
    coords(j, tm, tn, ksp, pb);
    const int par = j & 1;
    const int64_t Mq = GROUPED ? group_m(grp, pb) : M;
    const int64_t Nq = GROUPED ? group_n(grp, pb) : N;
    void* const Yq = GROUPED ? group_y(grp, pb) : Y;
    const float* const rq = GROUPED ? group_resid(grp, pb) : epi.resid;
    const int64_t ybase = (((int64_t)ksp * Mq + (int64_t)tm * BM) * Nq + (int64_t)tn * BN) * 4;
    const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<char*>(Yq) + ybase, (short)0, kBigRange, kRsrcWord3);
    // The tile's epilogue form: the kernel's own, or (mixed groups) its
    // problem's, uniform over the workgroup. For a fixed form these fold to
    // constants.
    constexpr bool kMixed = EPI == kEpiMixed;
    const int ek = kMixed ? group_kind(grp, pb) : EPI;
    const bool ebias = kMixed ? group_bias(grp, pb) : BIAS;
    const bool efma = kMixed ? group_fma(grp, pb) : epi.gate_fma != 0;
    constexpr bool kMayX = kMixed || EPI == SDQ_EPI_GATED || EPI == SDQ_EPI_RESID;
    const bool has_x = kMayX && (ek == SDQ_EPI_GATED || ek == SDQ_EPI_RESID);
    (void)ebias;
    (void)efma;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        has_x ? const_cast<float*>(rq) + (ybase >> 2) : static_cast<float*>(Yq), (short)0,
        has_x ? kBigRange : 0, kRsrcWord3);
    // 32-bit row / column checks: M <= 2^30, and N fits the 32-bit offsets
    const int mrow0 = tm * BM + wrow + rr;
    const int ncol0 = tn * BN + wcol + 4 * rc;
    const int M32 = (int)Mq, N32 = (int)Nq;
    // Opaque copy of the lane's offset: keeps the compiler from hoisting the
    // per-row output offsets out of the tile loop (they would stay live
    // across the main loop and spill).
    const int ldyq = GROUPED ? N32 * 4 : ldy4;
    int vlane = GROUPED ? (wrow + rr) * ldyq + (wcol + 4 * rc) * 4 : voff_lane;
    asm volatile("" : "+v"(vlane));
    // GELU: running max |Y| of the lane's rows over its columns (for the
    // next GEMM's activation quantizer); NaN never wins, as in the
    // quantizer's own max.
    constexpr bool kRowMax = EPI == SDQ_EPI_GELU;
    float rm[kRowMax ? FM : 1][4] = {};
#pragma unroll
    for (int a = 0; a < FN; a++) {
      const int cl = wcol + a * 32 + 4 * rc;  // tile column of this lane's chunk
      const bool n_ok = ncol0 + a * 32 < N32;
      const float4 s4 = *reinterpret_cast<const float4*>(&colb[par][0][cl]);
      const float4 b4 = *reinterpret_cast<const float4*>(&colb[par][1][cl]);
      const float4 g4 = *reinterpret_cast<const float4*>(&colb[par][2][cl]);
      // The residual of this column chunk's rows, all loads issued before
      // the first use: one memory latency per chunk column instead of one
      // per store. Each lane reads only the elements it writes afterwards,
      // so this is safe when the residual is Y itself.
      v4f xa[kMayX ? FM : 1][4];
      if (kMayX && has_x) {
#pragma unroll
        for (int b = 0; b < FM; b++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int rl = b * 32 + 8 * i;
            const bool ok = n_ok && (mrow0 + rl < M32);
            xa[b][i] = __builtin_amdgcn_raw_buffer_load_b128(
                xr, ok ? vlane + rl * ldyq + a * 128 : kOutOfRange, 0, 0);
          }
      }
#pragma unroll
      for (int b = 0; b < FM; b++) {
        // transpose the block: MFMA layout -> scratch -> row layout. Its
        // four 16x16 quarters: lane holds block row 16hb + (l & 15), 4-column
        // chunk 4ha + (l >> 4).
        // With 2 KB of scratch the block goes through in two halves of 16
        // rows (slots 0 and 1 each time); a wave's LDS accesses run in
        // order, so the second half's writes follow the first half's reads.
        v4i t4[4];
#pragma unroll
        for (int h = 0; h < kHalves; h++) {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const int ha = q >> 1, hb = q & 1;
            if (kHalves == 2 && hb != h) continue;
            const int row = 16 * hb + (lane & 15), chunk = 4 * ha + (lane >> 4);
            const int slot = kHalves == 2 ? ((row >> 3) & 1) : (row >> 3);
            *reinterpret_cast<v4i*>(scr + slot * kSlot + (row & 7) * 128 +
                                    ((chunk ^ (row & 7)) * 16)) = acc16[2 * a + ha][2 * b + hb];
          }
#pragma unroll
          for (int i = 0; i < 4 / kHalves; i++) {
            const int slot = kHalves == 2 ? i : i + h * 4;
            t4[h * (4 / kHalves) + i] =
                *reinterpret_cast<const v4i*>(scr + slot * kSlot + rr * 128 + ((rc ^ rr) * 16));
          }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int rl = b * 32 + 8 * i;  // block row offset of this store
          const bool ok = n_ok && (mrow0 + rl < M32);
          // All offsets in the VGPR, soffset 0: the compiler then inserts
          // the wait states a wide store's data VGPRs need before reuse.
          const int voff = ok ? vlane + rl * ldyq + a * 128 : kOutOfRange;
          if constexpr (EPI == SDQ_EPI_ACC) {
            __builtin_amdgcn_raw_buffer_store_b128(t4[i], yr, voff, 0, kStreamStore);
          } else {
            const float as_m = rowb[par][wrow + rl + rr];
            const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
            const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
            const float gv[4] = {g4.x, g4.y, g4.z, g4.w};
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const float sc = as_m * sv[r];
              const float af = (float)t4[i][r];
              v[r] = af * sc;  // K > 0 here (the launcher requires it)
            }
            if constexpr (!kMixed) {
              if constexpr (BIAS) {
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = v[r] + bv[r];
              }
              if constexpr (EPI == SDQ_EPI_GELU) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                  v[r] = gelu_tanh(v[r]);
                  const float av = ok ? fabsf(v[r]) : 0.f;
                  rm[b][i] = rm[b][i] < av ? av : rm[b][i];
                }
              } else if constexpr (EPI == SDQ_EPI_GATED || EPI == SDQ_EPI_RESID) {
                const v4f x = xa[b][i];
                if constexpr (EPI == SDQ_EPI_RESID) {
#pragma unroll
                  for (int r = 0; r < 4; r++) v[r] = x[r] + v[r];
                } else {
                  // both forms, then a select on the uniform flag: no branch
                  // between the loads and their uses
#pragma unroll
                  for (int r = 0; r < 4; r++) {
                    const float f = __builtin_fmaf(v[r], gv[r], x[r]);
                    const float p = v[r] * gv[r];
                    const float q = x[r] + p;
                    v[r] = epi.gate_fma ? f : q;
                  }
                }
              }
            } else {
              if (ebias) {
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = v[r] + bv[r];
              }
              if (ek == SDQ_EPI_GELU) {
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = gelu_tanh(v[r]);
              } else if (has_x) {
                const v4f x = xa[b][i];
                if (ek == SDQ_EPI_RESID) {
#pragma unroll
                  for (int r = 0; r < 4; r++) v[r] = x[r] + v[r];
                } else {
#pragma unroll
                  for (int r = 0; r < 4; r++) {
                    const float f = __builtin_fmaf(v[r], gv[r], x[r]);
                    const float p = v[r] * gv[r];
                    const float q = x[r] + p;
                    v[r] = efma ? f : q;
                  }
                }
              }
            }
            const v4f out = {v[0], v[1], v[2], v[3]};
            __builtin_amdgcn_raw_buffer_store_b128(out, yr, voff, 0, kStreamStore);
          }
        }
        // keep the scheduler from hoisting every block's operands at once
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (kRowMax) {
      // Lanes rr*8 .. rr*8+7 hold the same rows: reduce over them, then
      // one lane per row writes the wave's column chunk tn*WN + wn.
      if (epi.rmax) {
#pragma unroll
        for (int b = 0; b < FM; b++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float m = rm[b][i];
#pragma unroll
            for (int d = 1; d < 8; d *= 2) {
              const float o = __shfl_xor(m, d);
              m = m < o ? o : m;
            }
            const int row = mrow0 + b * 32 + 8 * i;
            if (rc == 0 && row < M32)
              epi.rmax[(int64_t)row * epi.rmax_stride + tn * WN + wn] = m;
          }
      }
    }
  }
  // the cursor's zero-range loads past the end still land in LDS
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
}

// ---------------------------------------------------------------------------
// Skinny kernel (M <= 32*FMS, FMS <= 8): one workgroup per 32 weight rows;
// its SPLIT waves stride over K, each streaming 1 KB weight fragments
// straight from HBM into VGPRs (and the small activation panel from L2),
// two k-fragments per group with the next group's loads in flight while
// the current one multiplies; then the partial int32 accumulators are
// summed through LDS in a fixed order (exact, so the order does not matter
// anyway). Small M is latency-bound on the tiled kernels (a 128x128 tile
// walks all of K alone); here every CU that holds a workgroup streams a
// quarter of K per wave.
template <int FMS, int SPLIT, int D>
__global__ void __launch_bounds__(SPLIT * 64)
qgemm_skinny(const int8_t* __restrict__ wt, const float* __restrict__ bs,
             const int8_t* __restrict__ at, const float* __restrict__ as, int64_t M, int64_t N,
             int64_t KFp, EpiArgs epi, void* Y, int vec) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t rb = blockIdx.x;
  const int8_t* wp = wt + rb * KFp * 1024 + lane * 16;
  const int8_t* ap = at + lane * 16;

  v16i acc[FMS];
#pragma unroll
  for (int j = 0; j < FMS; j++) acc[j] = v16i{};

  constexpr int U = 2;  // k-fragments per group; KFp is a multiple of 8 = U * SPLIT
  static_assert(U * SPLIT == 8, "groups tile KFp exactly");
  const int64_t ngrp = KFp / (U * SPLIT);
  struct Grp {
    v4i a[U], b[U][FMS];
  };
  auto load = [&](int64_t g, Grp& x) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t kb = w + (g * U + u) * SPLIT;
      x.a[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + kb * 1024));
#pragma unroll
      for (int j = 0; j < FMS; j++)
        x.b[u][j] = *reinterpret_cast<const v4i*>(ap + (j * KFp + kb) * 1024);
    }
  };
  auto mma = [&](const Grp& x) {
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int j = 0; j < FMS; j++)
        acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x.a[u], x.b[u][j], acc[j], 0, 0, 0);
  };
  // D groups in flight: group g + D loads while groups g+1 .. g+D-1 multiply
  Grp c[D];
#pragma unroll
  for (int d = 0; d < D; d++)
    if (d < ngrp) load(d, c[d]);
  for (int64_t g = 0; g < ngrp; g += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      if (g + d < ngrp) {
        mma(c[d]);
        if (g + d + D < ngrp) load(g + d + D, c[d]);
      }
    }
  }

  __shared__ int red[SPLIT][16][64];
  const int64_t n_lane = rb * 32 + (lane >> 5) * 4;
#pragma unroll
  for (int j = 0; j < FMS; j++) {
#pragma unroll
    for (int r = 0; r < 16; r++) red[w][r][lane] = acc[j][r];
    __syncthreads();
    if (w == 0) {
      v16i s;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        int t = red[0][r][lane];
#pragma unroll
        for (int ww = 1; ww < SPLIT; ww++) t += red[ww][r][lane];
        s[r] = t;
      }
      const int64_t m = j * 32 + (lane & 31);
      const float as_m = (m < M) ? as[m] : 0.f;
      store_block(s, m, n_lane, M, N, as_m, bs, epi, Y, vec);
    }
    __syncthreads();
  }
}

// Tiny M (M <= kQinMaxM rows): the skinny kernel (one row fragment) with the
// activation quantizer folded in. Every workgroup quantizes the few rows of
// A itself, with the quantizer's exact steps (max |a| with NaN never
// winning, sc = mx/127 or 1, inv = 1/sc, quant_one), into LDS (M rows of
// KFp*32 bytes, zero-padded values beyond K): M*K*4 bytes read from L2 per
// workgroup (12 KB at M = 1, K = 3072), so the call is one launch with no
// quantized-activation round trip.
template <int SPLIT, int D>
__global__ void __launch_bounds__(SPLIT * 64)
qgemm_skinny_qin(const int8_t* __restrict__ wt, const float* __restrict__ bs,
                 const float* __restrict__ A, int64_t M, int64_t K, int64_t N, int64_t KFp,
                 EpiArgs epi, void* Y, int vec, int avec) {
  extern __shared__ __attribute__((aligned(16))) int8_t aqs[];  // [M][KFp * 32]
  __shared__ float rmx[SPLIT][kQinMaxM];
  __shared__ float rsc[kQinMaxM], rinv[kQinMaxM];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  constexpr int NT = SPLIT * 64;
  const int64_t KB = KFp * 32;  // bytes per quantized row
  const int Mi = (int)M;
  for (int r = 0; r < Mi; r++) {
    const float* row = A + r * K;
    float mx = 0.f;
    if (avec) {
      for (int64_t k4 = tid; k4 < K / 4; k4 += NT) {
        const float4 v = reinterpret_cast<const float4*>(row)[k4];
        const float a[4] = {fabsf(v.x), fabsf(v.y), fabsf(v.z), fabsf(v.w)};
#pragma unroll
        for (int e = 0; e < 4; e++) mx = (mx < a[e]) ? a[e] : mx;
      }
    } else {
      for (int64_t k = tid; k < K; k += NT) {
        const float a = fabsf(row[k]);
        mx = (mx < a) ? a : mx;
      }
    }
#pragma unroll
    for (int d = 1; d < 64; d *= 2) {
      const float o = __shfl_xor(mx, d);
      mx = (mx < o) ? o : mx;
    }
    if (lane == 0) rmx[w][r] = mx;
  }
  __syncthreads();
  if (tid < Mi) {
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < SPLIT; i++) mx = (mx < rmx[i][tid]) ? rmx[i][tid] : mx;
    float sc = mx / 127.f;
    if (sc == 0.f) sc = 1.f;
    rsc[tid] = sc;
    rinv[tid] = 1.f / sc;
  }
  __syncthreads();
  for (int r = 0; r < Mi; r++) {
    const float* row = A + r * K;
    const float inv = rinv[r];
    for (int64_t k4 = tid; k4 < KB / 4; k4 += NT) {
      uint32_t x = 0;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int64_t k = 4 * k4 + e;
        const float v = k < K ? row[k] : 0.f;
        x |= (uint32_t)(uint8_t)(int8_t)quant_one(v, inv) << (8 * e);
      }
      *reinterpret_cast<uint32_t*>(aqs + r * KB + 4 * k4) = x;
    }
  }
  __syncthreads();

  const int64_t rb = blockIdx.x;
  const int8_t* wp = wt + rb * KFp * 1024 + lane * 16;
  const int arow = lane & 31;
  const int8_t* ap = aqs + (arow < Mi ? arow : 0) * KB + 16 * (lane >> 5);
  v16i acc = v16i{};
  constexpr int U = 2;
  static_assert(U * SPLIT == 8, "groups tile KFp exactly");
  const int64_t ngrp = KFp / (U * SPLIT);
  struct Grp {
    v4i a[U], b[U];
  };
  auto load = [&](int64_t g, Grp& x) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t kb = w + (g * U + u) * SPLIT;
      x.a[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + kb * 1024));
      x.b[u] = arow < Mi ? *reinterpret_cast<const v4i*>(ap + kb * 32) : v4i{};
    }
  };
  auto mma = [&](const Grp& x) {
#pragma unroll
    for (int u = 0; u < U; u++)
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(x.a[u], x.b[u], acc, 0, 0, 0);
  };
  // D groups in flight: group g + D loads while groups g+1 .. g+D-1 multiply
  Grp c[D];
#pragma unroll
  for (int d = 0; d < D; d++)
    if (d < ngrp) load(d, c[d]);
  for (int64_t g = 0; g < ngrp; g += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      if (g + d < ngrp) {
        mma(c[d]);
        if (g + d + D < ngrp) load(g + d + D, c[d]);
      }
    }
  }

  __shared__ int red[SPLIT][16][64];
#pragma unroll
  for (int r = 0; r < 16; r++) red[w][r][lane] = acc[r];
  __syncthreads();
  if (w == 0) {
    v16i sacc;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      int t = red[0][r][lane];
#pragma unroll
      for (int ww = 1; ww < SPLIT; ww++) t += red[ww][r][lane];
      sacc[r] = t;
    }
    const int64_t m = lane & 31;
    const float as_m = (m < M) ? rsc[m] : 0.f;
    store_block(sacc, m, rb * 32 + (lane >> 5) * 4, M, N, as_m, bs, epi, Y, vec);
  }
}

template <int BN, int BM, int WN, int WM, int KS, int STAGES>
hipError_t run_tiled(const int8_t* wt, const float* bs, const int8_t* at, const float* as,
                     int64_t M, int64_t N, int64_t KFp, const EpiArgs& epi, void* Y, int vec,
                     hipStream_t s) {
  const int tiles_n = (int)ceil_div(N, BN), tiles_m = (int)ceil_div(M, BM);
  const int64_t T = (int64_t)tiles_n * tiles_m;
  if (T <= 0) return hipSuccess;
  if (T > 0x3FFFFFFF) return hipErrorInvalidValue;  // the kernel counts tiles in 32 bits
  if (KFp % KS != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL((qgemm_tiled<BN, BM, WN, WM, KS, STAGES>), dim3((unsigned)T),
                     dim3(WN * WM * 64), 0, s, wt, bs, at, as, M, N, KFp, tiles_n, tiles_m, epi, Y,
                     vec);
  return hipGetLastError();
}

template <int BN, int BM, int WN, int WM, int KS, int STAGES, int OCC>
hipError_t run_persist(const int8_t* wt, const ColOps& cols, const int8_t* at, const float* as,
                       int64_t M, int64_t N, int64_t KFp, const EpiArgs& epi, void* Y,
                       int max_groups, hipStream_t s, int splits = 1) {
  const int tiles_n = (int)ceil_div(N, BN), tiles_m = (int)ceil_div(M, BM);
  const int64_t T = (int64_t)tiles_n * tiles_m * splits;
  if (T <= 0) return hipSuccess;
  if (T > 0x3FFFFFFF) return hipErrorInvalidValue;  // the kernel counts work items in 32 bits
  // K > 0 and at least STAGES stages per work item: the epilogue has no
  // K == 0 case
  if (splits < 1 || KFp % (KS * splits) != 0 || KFp / splits / KS < STAGES || epi.kzero)
    return hipErrorInvalidValue;
  int G = (int)(T < max_groups ? T : max_groups);
  if (G >= 8) G &= ~7;  // keeps virtual block ids on their XCD
  if (splits > 1) {
    if (epi.kind != SDQ_EPI_ACC) return hipErrorInvalidValue;
    hipLaunchKernelGGL((qgemm_persist<BN, BM, WN, WM, KS, STAGES, OCC, SDQ_EPI_ACC, false, true>),
                       dim3((unsigned)G), dim3(WN * WM * 64), 0, s, wt, cols, at, as, M, N, KFp,
                       tiles_n, tiles_m, epi, Y, splits, NoGroup{});
    return hipGetLastError();
  }
#define SDQ_LAUNCH_PERSIST(K, B)                                                                  \
  hipLaunchKernelGGL((qgemm_persist<BN, BM, WN, WM, KS, STAGES, OCC, K, B, false>),              \
                     dim3((unsigned)G), dim3(WN * WM * 64), 0, s, wt, cols, at, as, M, N, KFp,  \
                     tiles_n, tiles_m, epi, Y, 1, NoGroup{})
#define SDQ_LAUNCH_PERSIST_B(K)    \
  if (epi.bias)                    \
    SDQ_LAUNCH_PERSIST(K, true);   \
  else                             \
    SDQ_LAUNCH_PERSIST(K, false)
  switch (epi.kind) {
    case SDQ_EPI_NONE: SDQ_LAUNCH_PERSIST_B(SDQ_EPI_NONE); break;
    case SDQ_EPI_GELU: SDQ_LAUNCH_PERSIST_B(SDQ_EPI_GELU); break;
    case SDQ_EPI_GATED: SDQ_LAUNCH_PERSIST_B(SDQ_EPI_GATED); break;
    case SDQ_EPI_RESID: SDQ_LAUNCH_PERSIST_B(SDQ_EPI_RESID); break;
    case SDQ_EPI_ACC: SDQ_LAUNCH_PERSIST(SDQ_EPI_ACC, false); break;
    default: return hipErrorInvalidValue;
  }
#undef SDQ_LAUNCH_PERSIST_B
#undef SDQ_LAUNCH_PERSIST
  return hipGetLastError();
}

// One launch of the 128x128 persistent kernel over the tiles of several
// problems (GemmGroup): the same per-tile work as separate launches, without
// the partly empty rounds and launch gaps of many small ones.
hipError_t run_persist_group(GemmGroup& g, int64_t KFp, const EpiArgs& epi, float* sink,
                             int cu_count, hipStream_t s) {
  constexpr int BN = 128, BM = 128, KS = 2, STAGES = 4;
  if (g.count < 1 || g.count > kMaxGemmGroup || KFp % KS != 0 || KFp / KS < STAGES ||
      epi.kzero || epi.rmax || !sink)
    return hipErrorInvalidValue;
  int64_t total = 0;
  const GemmProblem& p0 = g.p[0];
  bool uniform = true;  // one epilogue form for every problem
  for (int i = 0; i < g.count; i++) {
    GemmProblem& p = g.p[i];
    const bool kind_ok = p.kind == SDQ_EPI_NONE || p.kind == SDQ_EPI_GELU ||
                         (p.kind == SDQ_EPI_GATED && p.gate && p.resid) ||
                         (p.kind == SDQ_EPI_RESID && p.resid);
    if (p.M <= 0 || p.N <= 0 || !p.wt || !p.scale || !p.at || !p.as || !p.Y || !kind_ok)
      return hipErrorInvalidValue;
    uniform = uniform && p.kind == p0.kind && (p.bias != nullptr) == (p0.bias != nullptr) &&
              (p.kind != SDQ_EPI_GATED || p.gate_fma == p0.gate_fma);
    p.tiles_n = (int)ceil_div(p.N, BN);
    p.tiles_m = (int)ceil_div(p.M, BM);
    p.tile0 = (int)total;
    total += (int64_t)p.tiles_n * p.tiles_m;
  }
  if (total > 0x7FFFFFFF / 2) return hipErrorInvalidValue;
  g.total = (int)total;
  const int64_t max_groups = 2 * (int64_t)(cu_count > 0 ? cu_count : 256);
  int G = (int)(total < max_groups ? total : max_groups);
  if (G >= 8) G &= ~7;
  const ColOps cols{p0.scale, p0.bias, p0.gate};
  EpiArgs ea = epi;
  ea.kind = uniform ? p0.kind : kEpiMixed;
  ea.gate_fma = p0.gate_fma;
  const bool bias = p0.bias != nullptr;
#define SDQ_LAUNCH_GROUP(K, B)                                                                    \
  hipLaunchKernelGGL((qgemm_persist<BN, BM, 2, 2, KS, STAGES, 2, K, B, false, true>),            \
                     dim3((unsigned)G), dim3(256), 0, s, p0.wt, cols, p0.at, p0.as,               \
                     (int64_t)p0.M, (int64_t)p0.N, KFp, p0.tiles_n, p0.tiles_m, ea,               \
                     static_cast<void*>(sink), 1, g)
#define SDQ_LAUNCH_GROUP_B(K)   \
  if (bias)                     \
    SDQ_LAUNCH_GROUP(K, true);  \
  else                          \
    SDQ_LAUNCH_GROUP(K, false)
  switch (ea.kind) {
    case SDQ_EPI_NONE: SDQ_LAUNCH_GROUP_B(SDQ_EPI_NONE); break;
    case SDQ_EPI_GELU: SDQ_LAUNCH_GROUP_B(SDQ_EPI_GELU); break;
    case SDQ_EPI_GATED: SDQ_LAUNCH_GROUP_B(SDQ_EPI_GATED); break;
    case SDQ_EPI_RESID: SDQ_LAUNCH_GROUP_B(SDQ_EPI_RESID); break;
    case kEpiMixed: SDQ_LAUNCH_GROUP(kEpiMixed, false); break;  // bias per problem
    default: return hipErrorInvalidValue;
  }
#undef SDQ_LAUNCH_GROUP_B
#undef SDQ_LAUNCH_GROUP
  return hipGetLastError();
}

// Split-K reduction: Y[m, n..n+3] = epilogue(sum_s part[s][m][n..n+3]),
// the same fp32 steps as the GEMM epilogues (the int32 sum is exact).
template <int EPI, bool BIAS>
__global__ void __launch_bounds__(256)
splitk_reduce(const int* __restrict__ part, int S, int64_t M, int64_t N,
              const float* __restrict__ as, const float* __restrict__ bs, EpiArgs epi, void* Y) {
  const int64_t n4 = N / 4;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * n4) return;
  const int64_t m = idx / n4, n = (idx - m * n4) * 4;
  v4i acc = *reinterpret_cast<const v4i*>(part + m * N + n);
  for (int s = 1; s < S; s++) acc += *reinterpret_cast<const v4i*>(part + (s * M + m) * N + n);
  if constexpr (EPI == SDQ_EPI_ACC) {
    *reinterpret_cast<v4i*>(static_cast<int*>(Y) + m * N + n) = acc;
    return;
  } else {
    const float as_m = as[m];
    const v4f s4 = *reinterpret_cast<const v4f*>(bs + n);
    v4f v;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float sc = as_m * s4[r];
      const float af = (float)acc[r];
      v[r] = af * sc;
    }
    if constexpr (BIAS) {
      const v4f b4 = *reinterpret_cast<const v4f*>(epi.bias + n);
#pragma unroll
      for (int r = 0; r < 4; r++) v[r] = v[r] + b4[r];
    }
    if constexpr (EPI == SDQ_EPI_GELU) {
#pragma unroll
      for (int r = 0; r < 4; r++) v[r] = gelu_tanh(v[r]);
    } else if constexpr (EPI == SDQ_EPI_GATED || EPI == SDQ_EPI_RESID) {
      const v4f x = *reinterpret_cast<const v4f*>(epi.resid + m * N + n);
      if constexpr (EPI == SDQ_EPI_RESID) {
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = x[r] + v[r];
      } else {
        const v4f g4 = *reinterpret_cast<const v4f*>(epi.gate + n);
        if (epi.gate_fma) {
#pragma unroll
          for (int r = 0; r < 4; r++) v[r] = __builtin_fmaf(v[r], g4[r], x[r]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const float p = v[r] * g4[r];
            v[r] = x[r] + p;
          }
        }
      }
    }
    *reinterpret_cast<v4f*>(static_cast<float*>(Y) + m * N + n) = v;
  }
}

hipError_t run_splitk_reduce(const int* part, int S, int64_t M, int64_t N, const float* as,
                             const float* bs, const EpiArgs& epi, void* Y, hipStream_t s) {
  const int64_t items = M * (N / 4);
  if (items <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)ceil_div(items, 256);
#define SDQ_LAUNCH_REDUCE(K, B)                                                              \
  hipLaunchKernelGGL((splitk_reduce<K, B>), dim3(blocks), dim3(256), 0, s, part, S, M, N, as, \
                     bs, epi, Y)
  const bool b = epi.bias != nullptr;
  switch (epi.kind) {
    case SDQ_EPI_NONE: if (b) SDQ_LAUNCH_REDUCE(SDQ_EPI_NONE, true); else SDQ_LAUNCH_REDUCE(SDQ_EPI_NONE, false); break;
    case SDQ_EPI_GELU: if (b) SDQ_LAUNCH_REDUCE(SDQ_EPI_GELU, true); else SDQ_LAUNCH_REDUCE(SDQ_EPI_GELU, false); break;
    case SDQ_EPI_GATED: if (b) SDQ_LAUNCH_REDUCE(SDQ_EPI_GATED, true); else SDQ_LAUNCH_REDUCE(SDQ_EPI_GATED, false); break;
    case SDQ_EPI_RESID: if (b) SDQ_LAUNCH_REDUCE(SDQ_EPI_RESID, true); else SDQ_LAUNCH_REDUCE(SDQ_EPI_RESID, false); break;
    case SDQ_EPI_ACC: SDQ_LAUNCH_REDUCE(SDQ_EPI_ACC, false); break;
    default: return hipErrorInvalidValue;
  }
#undef SDQ_LAUNCH_REDUCE
  return hipGetLastError();
}

// Groups in flight per wave in the skinny kernels (4 vs 2: equal within
// noise at M=1..64, 1-7% better at M=5..20 with long K).
constexpr int kSkinnyDepth = 4;

template <int FMS>
hipError_t run_skinny(const int8_t* wt, const float* bs, const int8_t* at, const float* as,
                      int64_t M, int64_t N, int64_t KFp, const EpiArgs& epi, void* Y, int vec,
                      hipStream_t s) {
  constexpr int SPLIT = 4;
  const int64_t blocks = ceil_div(N, 32);
  if (blocks <= 0) return hipSuccess;
  if (KFp % 8 != 0 || KFp < 8) return hipErrorInvalidValue;
  constexpr int D = FMS <= 2 ? kSkinnyDepth : 2;  // register budget of the wider groups
  hipLaunchKernelGGL((qgemm_skinny<FMS, SPLIT, D>), dim3((unsigned)blocks), dim3(SPLIT * 64), 0,
                     s, wt, bs, at, as, M, N, KFp, epi, Y, vec);
  return hipGetLastError();
}

hipError_t run_skinny_m(const int8_t* wt, const float* bs, const int8_t* at, const float* as,
                        int64_t M, int64_t N, int64_t KFp, const EpiArgs& epi, void* Y, int vec,
                        hipStream_t s) {
  switch (ceil_div(M, 32)) {
    case 1: return run_skinny<1>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case 2: return run_skinny<2>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case 3: return run_skinny<3>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case 4: return run_skinny<4>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case 5: return run_skinny<5>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case 6: return run_skinny<6>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case 7: return run_skinny<7>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case 8: return run_skinny<8>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool qin_fits(int64_t M, int64_t K, int64_t KFp) {
  // Every workgroup reads and quantizes M*K values first: worth it up to
  // M*K = 8192 (measured, N=18432: M=1 21.8 -> 12.6 us, M=2 22.3 -> 15.5,
  // M=4 22.6 -> 20.8 at K=3072; at M=4, K=14336 it loses, 30.6 -> 51).
  return M >= 1 && M <= kQinMaxM && K > 0 && M * K <= 8192 && M * KFp * 32 <= kQinMaxLds;
}

hipError_t launch_qgemm_qin(const int8_t* wt, const float* bs, const float* A, int64_t M,
                            int64_t K, int64_t N, int64_t KFp, const EpiArgs& epi, void* Y,
                            int vec, hipStream_t s) {
  if (!qin_fits(M, K, KFp) || KFp % 8 != 0 || epi.kzero) return hipErrorInvalidValue;
  const int64_t blocks = ceil_div(N, 32);
  if (blocks <= 0) return hipSuccess;
  const int avec = ((reinterpret_cast<uintptr_t>(A) & 15) == 0 && K % 4 == 0) ? 1 : 0;
  hipLaunchKernelGGL((qgemm_skinny_qin<4, kSkinnyDepth>), dim3((unsigned)blocks), dim3(4 * 64),
                     (unsigned)(M * KFp * 32), s, wt, bs, A, M, K, N, KFp, epi, Y, vec, avec);
  return hipGetLastError();
}

int gemm_cfg_bm(int cfg) {
  switch (cfg) {
    case kCfgSkinny: return 32;
    case kCfg128x128: return 128;
    case kCfg256x256: return 256;
    default: return 256;
  }
}

const char* gemm_cfg_name(int cfg) {
  switch (cfg) {
    case kCfgSkinny: return "skinny";
    case kCfg128x128: return "tile128x128";
    case kCfg256x256: return "tile256x256";
    default: return "?";
  }
}

int choose_gemm_cfg(int64_t M, int64_t N, int64_t KFp, int epi_kind, int cu_count) {
  if (const char* f = std::getenv("SDQ_FORCE_CFG")) {
    const int c = std::atoi(f);
    if (c >= kCfg128x128 && c < kCfgCount && M > 128) return c;
    if (c == kCfgSkinny && M <= kSkinnyMaxM) return c;
  }
  if (M <= 64) return kCfgSkinny;
  const int64_t t256 = ceil_div(M, 256) * ceil_div(N, 256);
  if (t256 >= 2 * (int64_t)(cu_count > 0 ? cu_count : 256)) return kCfg256x256;
  return kCfg128x128;
}

int gemm_rmax_chunks(int cfg, int64_t N) {
  // both persistent configs have two wave columns per tile
  if (cfg == kCfg128x128) return (int)ceil_div(N, 128) * 2;
  if (cfg == kCfg256x256) return (int)ceil_div(N, 256) * 2;
  return 0;
}

hipError_t launch_qgemm_group(GemmGroup& g, int64_t KFp, const EpiArgs& epi, float* sink,
                              int cu_count, hipStream_t s) {
  return run_persist_group(g, KFp, epi, sink, cu_count, s);
}

int64_t tail_split_rows(int64_t M, int64_t N, int cu_count) {
  // A last round of 256x256 tiles under half full: the rows of the full
  // rounds (whole m-tiles) run as 256x256 tiles, the rest as 128x128 tiles.
  if (std::getenv("SDQ_NO_TAIL")) return 0;
  const int64_t tn = ceil_div(N, 256), T = ceil_div(M, 256) * tn;
  const int64_t G = cu_count > 0 ? cu_count : 256;
  const int64_t full = (T / G) * G, tail = T - full;
  const int64_t Ma = (full / tn) * 256;
  return (tail > 0 && 2 * tail < G && Ma > 0 && Ma < M) ? Ma : 0;
}

int choose_splitk(int cfg, int64_t M, int64_t N, int64_t KFp, int cu_count) {
  // Long K on a grid that leaves workgroup slots idle: split K so the
  // 128x128 kernel's (tile, k-range) items fill up to its 2 slots per CU,
  // at most 4 ways, each item keeping >= 16 k-fragments. Measured at K =
  // 14336: N = 3072, M = 768 (144 tiles) 71 -> 58 us with S = 2 (288 items);
  // M = 157 (48 tiles) best at S = 4 (24 us; S = 8: 25-29 us).
  // SDQ_FORCE_SPLITK=S overrides the factor (1 = never split); a factor
  // that does not divide the k-fragments into >= 16 per item is lowered.
  if (cfg != kCfg128x128 || N % 4 != 0) return 1;
  int S = 0;
  if (const char* f = std::getenv("SDQ_FORCE_SPLITK")) S = std::atoi(f) < 1 ? 1 : std::atoi(f);
  if (S == 0) {
    if (KFp < 192) return 1;
    const int64_t T = ceil_div(M, 128) * ceil_div(N, 128);
    const int64_t per = 2 * (int64_t)(cu_count > 0 ? cu_count : 256) / T;
    S = per < 1 ? 1 : (per > 4 ? 4 : (int)per);
  }
  if (S > 8) S = 8;
  while (S > 1 && (KFp % (2 * S) != 0 || KFp / S < 16)) S--;
  return S;
}

hipError_t launch_qgemm(int cfg, const int8_t* wt, const float* bs, const int8_t* at,
                        const float* as, int64_t M, int64_t N, int64_t KFp, const EpiArgs& epi,
                        void* Y, int vec, const GemmAux& aux, hipStream_t s) {
  const ColOps cols{bs, aux.bias_pad, aux.gate_pad};
  // The persistent kernel addresses a tile's panels and output rows with
  // 32-bit buffer offsets.
  const bool persist = vec && aux.sink && !epi.kzero && KFp * 1024 * 8 <= 0x7FFFFFFF &&
                       N * 4 * 256 <= 0x7FFFFFF0;
  // Row maxima of a GELU output: written by the persistent kernels only
  // (not under split-K), one column chunk per wave column of each tile.
  if (aux.rmax_chunks) *aux.rmax_chunks = 0;
  if (aux.tail) *aux.tail = 0;
  const bool rmax = epi.rmax && epi.kind == SDQ_EPI_GELU && persist && aux.splitk <= 1 &&
                    (cfg == kCfg128x128 || cfg == kCfg256x256) &&
                    gemm_rmax_chunks(cfg, N) <= epi.rmax_stride;
  EpiArgs epi_r = epi;
  if (!rmax) epi_r.rmax = nullptr;
  else if (aux.rmax_chunks) *aux.rmax_chunks = gemm_rmax_chunks(cfg, N);
  switch (cfg) {
    case kCfgSkinny:
      if (M > kSkinnyMaxM) return hipErrorInvalidValue;
      return run_skinny_m(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case kCfg128x128:
      if (persist && aux.splitk > 1 && aux.part) {
        EpiArgs acc_epi = epi;
        acc_epi.kind = SDQ_EPI_ACC;
        hipError_t e = run_persist<128, 128, 2, 2, 2, 4, 2>(wt, cols, at, as, M, N, KFp, acc_epi,
                                                            aux.part, 2 * aux.cu_count, s,
                                                            aux.splitk);
        if (e != hipSuccess) return e;
        return run_splitk_reduce(aux.part, aux.splitk, M, N, as, bs, epi, Y, s);
      }
      if (persist)
        return run_persist<128, 128, 2, 2, 2, 4, 2>(wt, cols, at, as, M, N, KFp, epi_r, Y,
                                                    2 * aux.cu_count, s);
      return run_tiled<128, 128, 2, 2, 2, 4>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case kCfg256x256:
      if (persist) {
        // A last round of 256x256 tiles under half full: the rows of the
        // full rounds (whole m-tiles) run here, the rest as 128x128 tiles (a
        // quarter of the work each, two per CU) right after. Not with row
        // maxima (the two tile widths write different column chunks).
        const int64_t Ma = epi_r.rmax ? 0 : tail_split_rows(M, N, aux.cu_count);
        if (Ma > 0) {
          hipError_t e = run_persist<256, 256, 2, 4, 2, 4, 1>(wt, cols, at, as, Ma, N, KFp, epi_r,
                                                              Y, aux.cu_count, s);
          if (e != hipSuccess) return e;
          if (aux.tail) *aux.tail = 1;
          if (aux.mid && (e = hipEventRecord(aux.mid, s)) != hipSuccess) return e;
          EpiArgs et = epi_r;
          if (et.resid) et.resid += Ma * N;
          return run_persist<128, 128, 2, 2, 2, 4, 2>(
              wt, cols, at + (Ma / kFragRows) * KFp * kFragBytes, as + Ma, M - Ma, N, KFp, et,
              static_cast<char*>(Y) + Ma * N * 4, 2 * aux.cu_count, s);
        }
        return run_persist<256, 256, 2, 4, 2, 4, 1>(wt, cols, at, as, M, N, KFp, epi_r, Y,
                                                    aux.cu_count, s);
      }
      return run_tiled<256, 256, 2, 4, 2, 4>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sdq
