// Internal declarations shared by the sdq HIP translation units.
//
// Fragment layout ("frag layout") used for both operands in HBM:
//   an operand with R rows and K int8 columns is cut into 32-row x 32-byte
//   fragments; fragment (rb, kb) covers rows [32rb, 32rb+32) and columns
//   [32kb, 32kb+32). It occupies 1024 contiguous bytes at
//   ((rb * KFp) + kb) * 1024, and inside it lane l (0..63) owns the 16 bytes
//   at l*16, holding row 32rb + (l & 31), columns 32kb + 16(l >> 5) .. +15.
//   This is the per-lane A/B operand of v_mfma_i32_32x32x32_i8 (A and B use
//   the same k placement, so the exact int32 sum does not depend on which
//   k the hardware assigns to a byte), so a 1 KB fragment moves
//   global -> LDS -> VGPRs as one linear, conflict-free 16-byte-per-lane
//   copy; the persistent kernels read the two fragments of a 64-byte stage
//   as v_mfma_i32_16x16x64_i8 operands instead (16 rows each, one 16-byte
//   read per lane). Rows are padded to a multiple of the largest GEMM tile and KFp to
//   a multiple of 8 fragments (256 bytes of K) with zeros.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "sdq.h"

namespace sdq {

constexpr int kFragRows = 32;
constexpr int kFragK = 32;
constexpr int kFragBytes = 1024;
constexpr int kKFragAlign = 8;   // KFp is a multiple of this many fragments
constexpr int kRowAlign = 256;   // weight rows padded to this (largest BN)
constexpr int kColPad = 256;     // extra zero floats after padded column arrays

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }
inline int64_t kfrags_padded(int64_t K) {
  return round_up(ceil_div(K < 1 ? 1 : K, kFragK), kKFragAlign);
}

// Sets the thread-local error text and returns `code`.
int set_error(int code, const std::string& msg);
int hip_error(hipError_t e, const char* what);

#define SDQ_HIP(call)                                     \
  do {                                                    \
    hipError_t e_ = (call);                               \
    if (e_ != hipSuccess) return ::sdq::hip_error(e_, #call); \
  } while (0)

struct EpiArgs {
  int kind;
  int gate_fma;
  int kzero;  // K == 0: the product is +0 (the reference returns its zero-filled out)
  const float* bias;
  const float* gate;
  const float* resid;
  // GELU only (optional): rmax[row * rmax_stride + c] = max |Y[row, n]| over
  // the n of column chunk c (gemm_rmax_chunks chunks), for the next GEMM's
  // activation quantizer. Launchers that cannot write it report 0 chunks.
  float* rmax;
  int rmax_stride;
};

// ---- launchers (return hipError_t of the launch) -------------------------
// Activation quantizer: A [M,K] f32 row-major -> frag layout (rows padded to
// Mp, zero rows beyond M) + as[M]. The same launch copies bias / gate (when
// non-null) into the zero-padded column buffers bias_pad / gate_pad of CP
// floats that the persistent GEMM moves by LDS-DMA.
struct ColCopy {
  const float* bias;
  const float* gate;
  float* bias_pad;
  float* gate_pad;
  int64_t N, CP;
};
// Few rows (Mp / 8 units below a grid's worth) run the split form: one
// kernel writes per-(row, k-chunk) maxima to pmax, a second reduces them and
// quantizes; act_quant_pmax_floats gives pmax's size (0: single kernel).
int64_t act_quant_pmax_floats(int64_t Mp, int64_t KFp, int cu_count);
hipError_t launch_act_quant_frags(const float* A, int64_t M, int64_t K, int64_t Mp, int64_t KFp,
                                  int8_t* at, float* as, const ColCopy& cc, float* pmax,
                                  int cu_count, hipStream_t s);
// Several plain fragment-layout quantizations in one launch (single-kernel
// form only: act_quant_pmax_floats(Mp, KFp) == 0 for every segment). Segment
// i takes units (Mp / 8 workgroups) [unit0, next unit0 or total).
constexpr int kMaxQuantSegs = 16;
struct QuantSeg {
  const float* A;
  int64_t M, K, KFp;
  int vec;  // A 16-byte aligned and K % 4 == 0
  int8_t* at;
  float* as;
  ColCopy cc;
  int64_t unit0;
};
struct QuantSegs {
  QuantSeg s[kMaxQuantSegs];
  int count;
  int64_t total;
};
hipError_t launch_act_quant_segs(const QuantSegs& segs, hipStream_t s);
// mod_rows(layernorm(A)) as the quantized rows (the DiT's norm + modulation
// before q|k|v and the FFN, blocks.cpp:18-43 + ovi_dit.cpp:161-172): per-row
// (mean, 1/std) into st[M] (bit-exact serial sums), then the quantizer on the
// transformed values. shift / scale: [K] device vectors.
struct LnModArgs {
  const float2* st;
  const float* shift;
  const float* scale;
};
hipError_t launch_act_quant_frags_lnmod(const float* A, int64_t M, int64_t K, int64_t Mp,
                                        int64_t KFp, int8_t* at, float* as, const ColCopy& cc,
                                        const float* shift, const float* scale, float eps,
                                        float2* st, hipStream_t s);
// In place on L rows of stride ld (C columns): rmsnorm with weight w (w ==
// nullptr: none), then RoPE of each head's first nr pairs with the (cos, sin)
// table cs [L][nr] (cs == nullptr: no RoPE). inv: [L] scratch.
// One column block of strided rows for launch_rmsnorm_rope_segs: L rows of
// stride ld at x; w NULL = rotation only; cs NULL / nr 0 = no rotation; inv
// [L] floats of scratch when w is set.
struct RmsSeg {
  float* x;
  int64_t L, ld;
  const float* w;
  const float* cs;
  int nr;
  float* inv;
};
constexpr int kMaxRmsSegs = 4;
hipError_t launch_rmsnorm_rope_segs(const RmsSeg* segs, int nseg, int64_t C, int heads, float eps,
                                    hipStream_t s);
hipError_t launch_rmsnorm_rope(float* x, int64_t L, int64_t C, int64_t ld, const float* w,
                               float eps, int heads, const float* cs, int nr, float* inv,
                               hipStream_t s);
// Per-row (mean, 1/std) of blocks.cpp:18-43 into st[M] (bit-exact serial
// sums); rows of K floats, contiguous.
hipError_t launch_ln_stats(const float* A, int64_t M, int64_t K, float eps, float2* st,
                           hipStream_t s);
// y = fmaf(fl((x - mu)*inv), w, b) with st from launch_ln_stats (w, b
// nullable: 1, 0). x, y: [M, K] contiguous (may alias).
hipError_t launch_ln_apply(const float* x, int64_t M, int64_t K, const float2* st, const float* w,
                           const float* b, float* y, hipStream_t s);
// x[i] += y[i], i < n.
hipError_t launch_add(float* x, const float* y, int64_t n, hipStream_t s);
// One residual epilogue of a Linear applied to x from the Linear's plain
// output y (the NONE epilogue, bias included): GATED x = fma(y, g, x) (or
// x + fl(y*g)), RESID x = x + y.
struct ResidStep {
  const float* y;     // [M, N]
  const float* gate;  // [N] (GATED)
  int kind;           // SDQ_EPI_GATED or SDQ_EPI_RESID
  int gate_fma;
};
// x[M, N] = b(a(x)): two Linears' residual epilogues in order, from outputs
// computed apart; the same bits as the two GEMMs applying them one after the
// other. N % 4 == 0 and every array 16-byte aligned.
hipError_t launch_resid2(float* x, int64_t M, int64_t N, const ResidStep& a, const ResidStep& b,
                         hipStream_t s);
// y[M,N] = x[M,K] . w[K,N] (+ bias): one fmaf chain per output over k in
// order from +0, then + bias (sd::matmul's per-output steps).
hipError_t launch_linear_f32(const float* x, int64_t M, int64_t K, const float* w, int64_t N,
                             const float* bias, float* y, int cu_count, hipStream_t s);
// Attention, head_dim 128 (launch_sdpa rejects nothing else; the API checks):
// out[i, head cols] = softmax(q_i . k_j / sqrt(128)) v_j over j < Lk.
// batch > 1: `batch` sequences stacked along the rows (sequence b: query rows
// [b*Lq, (b+1)*Lq), key / value rows [b*Lk, (b+1)*Lk)), each attending only
// to its own keys.
// part (nullable): scratch of sdpa_part_floats floats; with it, few queries
// run as key splits (more workgroups) merged by a second kernel; without it,
// one workgroup walks all keys. cu_count: the device's CUs.
hipError_t launch_sdpa(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                       int64_t ldv, float* out, int64_t ldo, int64_t Lq, int64_t Lk, int heads,
                       hipStream_t s, int batch = 1, float* part = nullptr, int cu_count = 0);
// Key splits launch_sdpa uses for a sequence (1 = none), and the scratch
// floats they need for `batch` stacked sequences (0 = none).
int sdpa_splits(int64_t Lq, int64_t Lk, int heads, int cu_count);
int64_t sdpa_part_floats(int64_t Lq, int64_t Lk, int heads, int batch, int cu_count);
// Same output, with the row maxima already known: max_c rmax[row*rstride + c]
// over c < rchunks (e.g. written by the producing GEMM's epilogue), so A is
// read once.
hipError_t launch_act_quant_frags_premax(const float* A, int64_t M, int64_t K, int64_t Mp,
                                         int64_t KFp, int8_t* at, float* as, const ColCopy& cc,
                                         const float* rmax, int rchunks, int rstride,
                                         int cu_count, hipStream_t s);
// Same quantizer, row-major int8 output [M,K] (parity API).
hipError_t launch_act_quant_rowmajor(const float* A, int64_t M, int64_t K, int8_t* aq, float* as,
                                     hipStream_t s);
// Weight repack: q [N,K] row-major (device) + scale (device, aligned) ->
// frag layout with Np rows + scale padded with zeros to Np.
hipError_t launch_repack_weight(const int8_t* q, const float* scale, int64_t N, int64_t K,
                                int64_t Np, int64_t KFp, int8_t* frags, float* scale_out,
                                hipStream_t s);
// Inverse of the repack (export / round-trip check).
hipError_t launch_unpack_weight(const int8_t* frags, int64_t N, int64_t K, int64_t KFp,
                                int8_t* q, hipStream_t s);

// GEMM tile configurations.
enum GemmCfg : int {
  kCfgSkinny = 0,   // M <= kSkinnyMaxM: 32-row activation blocks, split-K waves
  kCfg128x128,      // BN=128, BM=128
  kCfg256x256,      // BN=256, BM=256
  kCfgCount
};
constexpr int64_t kSkinnyMaxM = 256;
int gemm_cfg_bm(int cfg);  // activation rows per tile (row padding of `at`)
const char* gemm_cfg_name(int cfg);
int choose_gemm_cfg(int64_t M, int64_t N, int64_t KFp, int epi_kind, int cu_count);
// Tiny M: the skinny GEMM quantizes A itself (one launch). qin_fits says
// whether M rows of K fit (M <= kQinMaxM, M*KFp*32 bytes of LDS <= kQinMaxLds).
constexpr int kQinMaxM = 4;
constexpr int64_t kQinMaxLds = 64 * 1024;
bool qin_fits(int64_t M, int64_t K, int64_t KFp);
hipError_t launch_qgemm_qin(const int8_t* wt, const float* bs, const float* A, int64_t M,
                            int64_t K, int64_t N, int64_t KFp, const EpiArgs& epi, void* Y,
                            int vec, hipStream_t s);
// Split-K factor for the 128x128 kernel at this shape (1 = no split).
int choose_splitk(int cfg, int64_t M, int64_t N, int64_t KFp, int cu_count);
// Rows of a 256x256 persistent launch that run as 256x256 tiles when the
// remaining rows go to a second, 128x128 launch; 0 = one launch.
int64_t tail_split_rows(int64_t M, int64_t N, int cu_count);

// Extra buffers of the persistent GEMM path: bias / gate copied into
// zero-padded buffers (nullptr when absent) so they can be moved by LDS-DMA,
// and a >= 1 KB scratch sink for the stores of masked lanes. sink == nullptr
// selects the non-persistent kernels.
struct GemmAux {
  const float* bias_pad;
  const float* gate_pad;
  float* sink;
  int cu_count;
  int splitk;  // choose_splitk's factor (1 = none)
  int* part;   // splitk x M x N int32 partial sums (splitk > 1)
  int* rmax_chunks;  // out (nullable): column chunks written to epi.rmax, 0 = none
  int* tail;         // out (nullable): 1 when a 256x256 launch handed its last rows to a
                     // second, 128x128 launch (two kernels ran), else 0
  hipEvent_t mid;    // nullable: recorded between those two launches (per-kernel timing)
};
// Grouped persistent GEMM: up to kMaxGemmGroup independent problems with
// the same K (KFp) in one launch of the 128x128 persistent kernel (each with
// its own epilogue kind, bias and gate form), their tiles walked as one
// list (problem p owns tiles [tile0, tile0 + tiles_n * tiles_m)). Each
// problem has its own
// weight, quantized activations (at / as, rows padded to 128), padded column
// operands (scale, bias, gate: as GemmAux / ColOps), residual and output.
constexpr int kMaxGemmGroup = 16;
struct GemmProblem {
  const int8_t* wt;
  const float* scale;
  const float* bias;
  const float* gate;
  const int8_t* at;
  const float* as;
  const float* resid;
  void* Y;
  int M, N, tiles_n, tiles_m, tile0;
  int kind;      // the problem's epilogue (SDQ_EPI_NONE / GELU / GATED / RESID)
  int gate_fma;  // GATED: fma form (else product, then add)
};
// A grouped launch whose problems differ in epilogue kind, bias presence or
// gate form: the kernel reads each tile's form from the problem table.
constexpr int kEpiMixed = 5;
struct GemmGroup {
  GemmProblem p[kMaxGemmGroup];
  int count;
  int total;  // tiles of all problems
};
// epi: kind, gate_fma (per-problem pointers come from the group; no row
// maxima). sink: >= 1 KB scratch (as GemmAux::sink).
hipError_t launch_qgemm_group(GemmGroup& g, int64_t KFp, const EpiArgs& epi, float* sink,
                              int cu_count, hipStream_t s);

// Column chunks of the row maxima a GELU launch of this config writes.
int gemm_rmax_chunks(int cfg, int64_t N);

hipError_t launch_qgemm(int cfg, const int8_t* wt, const float* bs, const int8_t* at,
                        const float* as, int64_t M, int64_t N, int64_t KFp, const EpiArgs& epi,
                        void* Y, int vec_ok, const GemmAux& aux, hipStream_t s);

}  // namespace sdq
