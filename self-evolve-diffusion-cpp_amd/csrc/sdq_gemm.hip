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
// and the ACTIVATION fragment its B operand (columns = m), so the 16x16 i32
// result C^T[n][m] lands as 4 consecutive n of one m per lane: lane l holds
// n = 4(l>>4) + r (r = 0..3), m = l & 15, i.e. a 16-byte row-contiguous
// store of Y[m, n..n+3].
#include "sdq_internal.h"

#pragma clang fp contract(off)

namespace sdq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float gelu_tanh(float v) {
  // nn.GELU(approximate='tanh'), src/model/ovi_dit.cpp:132-142.
  const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  return 0.5f * v * (1.f + tanhf(u));
}

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

// Epilogue for acc = C^T[n0..n0+3][m] of one lane.
__device__ __forceinline__ void store_out(const v4i acc, int64_t m, int64_t n0, int64_t M,
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

// ---------------------------------------------------------------------------
// Tiled kernel: one workgroup computes a BN (weight rows) x BM (activation
// rows) output tile. Each stage moves KS k-fragments of both panels
// global -> LDS with direct-to-LDS 16-byte loads (no VGPR staging), double
// buffered; WN x WM waves each own FN x FM 16x16 accumulator fragments.
template <int BN, int BM, int WN, int WM, int KS>
__global__ void __launch_bounds__(WN* WM * 64, 1)
qgemm_tiled(const int8_t* __restrict__ wt, const float* __restrict__ bs,
            const int8_t* __restrict__ at, const float* __restrict__ as, int64_t M, int64_t N,
            int64_t KFp, int tiles_n, int tiles_m, EpiArgs epi, void* Y, int vec) {
  constexpr int NW = WN * WM;
  constexpr int RBN = BN / 16, RBM = BM / 16;
  constexpr int FN = RBN / WN, FM = RBM / WM;
  constexpr int WFR = RBN * KS, AFR = RBM * KS, SFR = WFR + AFR;
  constexpr int WLD = WFR / NW, ALD = AFR / NW;  // load instructions per wave per stage
  constexpr int STAGE = SFR * 1024;
  static_assert(WFR % NW == 0 && AFR % NW == 0, "stage fragments must split evenly over waves");
  static_assert(NW % KS == 0, "waves must be a multiple of k-fragments per stage");
  __shared__ __attribute__((aligned(1024))) char lds[2 * STAGE];

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

  // ---- per-lane global offsets of this wave's loads (stage 0).
  // Stage fragment f = t*NW + w; W fragments first, then activation ones.
  // With NW % KS == 0 the k index of all of a wave's fragments is w % KS and
  // the row block advances by NW/KS per t.
  const uint32_t lane_off = (uint32_t)lane * 16u;
  const int64_t wbase = ((int64_t)(tn * RBN + w / KS) * KFp + (w % KS)) * 1024;
  const int64_t abase = ((int64_t)(tm * RBM + w / KS) * KFp + (w % KS)) * 1024;
  const int64_t tstride = (int64_t)(NW / KS) * KFp * 1024;

  v4i acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; i++)
#pragma unroll
    for (int j = 0; j < FM; j++) acc[i][j] = v4i{0, 0, 0, 0};

  const int nks = (int)(KFp / KS);

  auto issue = [&](int ks, char* buf) {
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

  issue(0, lds);
  for (int ks = 0; ks < nks; ks++) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (ks + 1 < nks) issue(ks + 1, lds + ((ks + 1) & 1) * STAGE);
    const char* cb = lds + (ks & 1) * STAGE;
#pragma unroll
    for (int kk = 0; kk < KS; kk++) {
      v4i a[FN], b[FM];
#pragma unroll
      for (int i = 0; i < FN; i++)
        a[i] = *reinterpret_cast<const v4i*>(cb + ((wn * FN + i) * KS + kk) * 1024 + lane_off);
#pragma unroll
      for (int j = 0; j < FM; j++)
        b[j] = *reinterpret_cast<const v4i*>(cb + WFR * 1024 + ((wm * FM + j) * KS + kk) * 1024 +
                                             lane_off);
#pragma unroll
      for (int i = 0; i < FN; i++)
#pragma unroll
        for (int j = 0; j < FM; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // ---- epilogue
  const int64_t mb = (int64_t)tm * BM + wm * FM * 16 + (lane & 15);
  const int64_t nb = (int64_t)tn * BN + wn * FN * 16 + (lane >> 4) * 4;
#pragma unroll
  for (int j = 0; j < FM; j++) {
    const int64_t m = mb + j * 16;
    const float as_m = (m < M) ? as[m] : 0.f;
#pragma unroll
    for (int i = 0; i < FN; i++) store_out(acc[i][j], m, nb + i * 16, M, N, as_m, bs, epi, Y, vec);
  }
}

// ---------------------------------------------------------------------------
// Skinny kernel (M <= 16*FMS): one workgroup per 16 weight rows; its SPLIT
// waves stride over K, each streaming 1 KB weight fragments straight from
// HBM into VGPRs, then the partial int32 accumulators are summed through LDS
// (exact, so the order does not matter).
template <int FMS, int SPLIT>
__global__ void __launch_bounds__(SPLIT * 64)
qgemm_skinny(const int8_t* __restrict__ wt, const float* __restrict__ bs,
             const int8_t* __restrict__ at, const float* __restrict__ as, int64_t M, int64_t N,
             int64_t KFp, EpiArgs epi, void* Y, int vec) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t rb = blockIdx.x;
  const int8_t* wp = wt + rb * KFp * 1024 + lane * 16;
  const int8_t* ap = at + lane * 16;

  v4i acc[FMS];
#pragma unroll
  for (int j = 0; j < FMS; j++) acc[j] = v4i{0, 0, 0, 0};

  constexpr int U = 4;
  int64_t kb = w;
  for (; kb + (int64_t)(U - 1) * SPLIT < KFp; kb += (int64_t)U * SPLIT) {
    v4i a[U], b[U][FMS];
#pragma unroll
    for (int u = 0; u < U; u++)
      a[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + (kb + u * SPLIT) * 1024));
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int j = 0; j < FMS; j++)
        b[u][j] = *reinterpret_cast<const v4i*>(ap + (j * KFp + kb + u * SPLIT) * 1024);
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int j = 0; j < FMS; j++)
        acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], b[u][j], acc[j], 0, 0, 0);
  }
  for (; kb < KFp; kb += SPLIT) {
    const v4i a = *reinterpret_cast<const v4i*>(wp + kb * 1024);
#pragma unroll
    for (int j = 0; j < FMS; j++) {
      const v4i b = *reinterpret_cast<const v4i*>(ap + (j * KFp + kb) * 1024);
      acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[j], 0, 0, 0);
    }
  }

  __shared__ v4i red[SPLIT][FMS][64];
#pragma unroll
  for (int j = 0; j < FMS; j++) red[w][j][lane] = acc[j];
  __syncthreads();
  if (w != 0) return;
  const int64_t n0 = rb * 16 + (lane >> 4) * 4;
#pragma unroll
  for (int j = 0; j < FMS; j++) {
    v4i s = red[0][j][lane];
#pragma unroll
    for (int ww = 1; ww < SPLIT; ww++) s += red[ww][j][lane];
    const int64_t m = j * 16 + (lane & 15);
    const float as_m = (m < M) ? as[m] : 0.f;
    store_out(s, m, n0, M, N, as_m, bs, epi, Y, vec);
  }
}

template <int BN, int BM, int WN, int WM, int KS>
hipError_t run_tiled(const int8_t* wt, const float* bs, const int8_t* at, const float* as,
                     int64_t M, int64_t N, int64_t KFp, const EpiArgs& epi, void* Y, int vec,
                     hipStream_t s) {
  const int tiles_n = (int)ceil_div(N, BN), tiles_m = (int)ceil_div(M, BM);
  const int64_t T = (int64_t)tiles_n * tiles_m;
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL((qgemm_tiled<BN, BM, WN, WM, KS>), dim3((unsigned)T), dim3(WN * WM * 64), 0,
                     s, wt, bs, at, as, M, N, KFp, tiles_n, tiles_m, epi, Y, vec);
  return hipGetLastError();
}

template <int FMS>
hipError_t run_skinny(const int8_t* wt, const float* bs, const int8_t* at, const float* as,
                      int64_t M, int64_t N, int64_t KFp, const EpiArgs& epi, void* Y, int vec,
                      hipStream_t s) {
  constexpr int SPLIT = 4;
  const int64_t blocks = ceil_div(N, 16);
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL((qgemm_skinny<FMS, SPLIT>), dim3((unsigned)blocks), dim3(SPLIT * 64), 0, s,
                     wt, bs, at, as, M, N, KFp, epi, Y, vec);
  return hipGetLastError();
}

}  // namespace

int gemm_cfg_bm(int cfg) {
  switch (cfg) {
    case kCfgSkinny1: return 16;
    case kCfgSkinny2: return 32;
    case kCfgSkinny4: return 64;
    case kCfg128x128: return 128;
    case kCfg256x256: return 256;
    default: return 256;
  }
}

const char* gemm_cfg_name(int cfg) {
  switch (cfg) {
    case kCfgSkinny1: return "skinny16";
    case kCfgSkinny2: return "skinny32";
    case kCfgSkinny4: return "skinny64";
    case kCfg128x128: return "tile128x128";
    case kCfg256x256: return "tile256x256";
    default: return "?";
  }
}

int choose_gemm_cfg(int64_t M, int64_t N, int cu_count) {
  if (M <= 16) return kCfgSkinny1;
  if (M <= 32) return kCfgSkinny2;
  if (M <= 64) return kCfgSkinny4;
  const int64_t t256 = ceil_div(M, 256) * ceil_div(N, 256);
  if (t256 >= 2 * (int64_t)(cu_count > 0 ? cu_count : 256)) return kCfg256x256;
  return kCfg128x128;
}

hipError_t launch_qgemm(int cfg, const int8_t* wt, const float* bs, const int8_t* at,
                        const float* as, int64_t M, int64_t N, int64_t KFp, const EpiArgs& epi,
                        void* Y, int vec, hipStream_t s) {
  switch (cfg) {
    case kCfgSkinny1: return run_skinny<1>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case kCfgSkinny2: return run_skinny<2>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case kCfgSkinny4: return run_skinny<4>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case kCfg128x128:
      return run_tiled<128, 128, 2, 2, 2>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    case kCfg256x256:
      return run_tiled<256, 256, 2, 4, 2>(wt, bs, at, as, M, N, KFp, epi, Y, vec, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sdq
