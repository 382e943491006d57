// C ABI of the sdq library (declared in include/sdq.h).
//
// Owns: per-device state, weight handles (fragment-layout copies of .sdcpp
// int8 weights in HBM), and a per-(device, stream) workspace holding the
// quantized activations of the call in flight. Every entry point reports
// failures as a status code plus a thread-local message and never throws
// (the reference's loader throws std::runtime_error, src/serde/sdcpp.cpp:27;
// its qgemm has no error path at all, src/core/qgemm.cpp:73-142).
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <map>
#include <mutex>
#include <new>
#include <set>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "sdq_internal.h"

// Scratch memory of sdq_qlinear_noalloc: a file-scope device array, one copy
// per GPU (each holds it until the process ends). In host code this name is
// only a stand-in for the symbol: host code uses the address that
// hipGetSymbolAddress returns for the current device (DevState::scratch),
// never the name itself.
static __device__ __align__(256) char scratch[SDQ_NOALLOC_SCRATCH_BYTES];

struct sdq_weight {
  int device;
  int64_t N, K, Np, KFp;
  int8_t* frags;  // (Np/32) * KFp * 1024 bytes
  float* scale;   // Np floats, zero padded
};

namespace sdq {

namespace {

thread_local std::string t_err;

struct DevState {
  bool ready = false;
  int cu_count = 0;
  hipDeviceProp_t prop{};
  char* scratch = nullptr;    // this device's copy of `scratch` (hipGetSymbolAddress)
  std::string scratch_err;    // why scratch is null, if it is
};

constexpr int kMaxDev = 64;
std::mutex g_mu;
DevState g_dev[kMaxDev];

struct Workspace {
  int8_t* at = nullptr;  // quantized activations, fragment layout
  size_t at_bytes = 0;
  float* as = nullptr;   // per-row activation scales
  size_t as_bytes = 0;
  float* cols = nullptr;  // [2][col_cap]: zero-padded bias, gate copies
  size_t col_cap = 0;
  float* sink = nullptr;  // 1 KB target of masked epilogue stores
  int* part = nullptr;    // split-K int32 partial sums
  size_t part_bytes = 0;
  float* pmax = nullptr;  // split quantizer's per-(row, k-chunk) maxima
  size_t pmax_bytes = 0;
  float* rmax = nullptr;  // row maxima of a GELU output (sdq_ffn's hidden state)
  size_t rmax_bytes = 0;
  float2* st = nullptr;  // layernorm row statistics (mean, 1/std)
  size_t st_bytes = 0;
  float* rinv = nullptr;  // rmsnorm 1/rms per row
  size_t rinv_bytes = 0;
  char* grp = nullptr;  // sdq_qlinear_group's per-item scratch
  size_t grp_bytes = 0;
  float* sdpa_part = nullptr;  // attention key splits' partial outputs and states
  size_t sdpa_part_bytes = 0;
};
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ---- optional per-kernel event timing (sdq_profile_begin/end) ----
struct ProfRec {
  std::string name;
  hipEvent_t a, b;
};
thread_local bool t_prof = false;
thread_local std::vector<ProfRec> t_recs;

hipEvent_t prof_mark(hipStream_t s) {
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  if (hipEventRecord(e, s) != hipSuccess) {
    (void)hipEventDestroy(e);
    return nullptr;
  }
  return e;
}

// Profiling marks not handed to the records (an error return).
void drop_events(std::initializer_list<hipEvent_t> evs) {
  for (hipEvent_t e : evs)
    if (e) (void)hipEventDestroy(e);
}

int current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return hip_error(e, "hipGetDevice");
  if (*dev < 0 || *dev >= kMaxDev) return set_error(SDQ_ERR_NODEV, "device index out of range");
  return SDQ_OK;
}

int ensure_device(int dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  DevState& d = g_dev[dev];
  if (d.ready) return SDQ_OK;
  hipError_t e = hipGetDeviceProperties(&d.prop, dev);
  if (e != hipSuccess) return hip_error(e, "hipGetDeviceProperties");
  if (std::strncmp(d.prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(SDQ_ERR_NODEV, std::string("sdq kernels are built for gfx950, device is ") +
                                        d.prop.gcnArchName);
  d.cu_count = d.prop.multiProcessorCount;
  // The no-alloc entry point's scratch on this device (current here): looked
  // up once; a failure only disables that entry point.
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e == hipSuccess && p) {
    d.scratch = static_cast<char*>(p);
  } else {
    (void)hipGetLastError();
    d.scratch_err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
  }
  d.ready = true;
  return SDQ_OK;
}

// Grows (never shrinks) the workspace of (dev, stream). A buffer that is
// replaced may still be read by work queued on `stream`, so the stream is
// drained before the old buffer is freed. A stream that is capturing a graph
// can be neither drained nor given new memory: the call is refused with an
// error that leaves the capture intact (a call of the same size or larger on
// the stream before the capture grows it in advance).
int grow(hipStream_t s, void** p, size_t* have, size_t need) {
  if (*have >= need) return SDQ_OK;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &st);
  if (e != hipSuccess) return hip_error(e, "hipStreamIsCapturing");
  if (st != hipStreamCaptureStatusNone)
    return set_error(SDQ_ERR_INVALID,
                     "the stream's workspace would have to grow while the stream captures a "
                     "graph: make the same call once on this stream before the capture");
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize");
  if (*p) (void)hipFree(*p);
  *p = nullptr;
  *have = 0;
  e = hipMalloc(p, need);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return set_error(SDQ_ERR_NOMEM, "workspace allocation of " + std::to_string(need) +
                                        " bytes failed");
  }
  *have = need;
  return SDQ_OK;
}

int workspace(int dev, hipStream_t s, size_t at_bytes, size_t as_bytes, size_t col_cap,
              size_t part_bytes, size_t pmax_bytes, Workspace** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  Workspace& w = g_ws[{dev, s}];
  int rc = grow(s, reinterpret_cast<void**>(&w.at), &w.at_bytes, at_bytes);
  if (!rc) rc = grow(s, reinterpret_cast<void**>(&w.as), &w.as_bytes, as_bytes);
  size_t cb = w.col_cap * 2 * sizeof(float);
  if (!rc && cb < col_cap * 2 * sizeof(float)) {
    rc = grow(s, reinterpret_cast<void**>(&w.cols), &cb, col_cap * 2 * sizeof(float));
    if (!rc) w.col_cap = col_cap;
  }
  if (!rc && !w.sink) {
    size_t have = 0;
    rc = grow(s, reinterpret_cast<void**>(&w.sink), &have, 4096);
  }
  if (!rc && part_bytes) rc = grow(s, reinterpret_cast<void**>(&w.part), &w.part_bytes, part_bytes);
  if (!rc && pmax_bytes) rc = grow(s, reinterpret_cast<void**>(&w.pmax), &w.pmax_bytes, pmax_bytes);
  if (rc) return rc;
  *out = &w;
  return SDQ_OK;
}

// A float buffer of the (device, stream) workspace (member buf / have),
// grown to at least `bytes`.
int ws_floats(int dev, hipStream_t s, float* Workspace::*buf, size_t Workspace::*have,
              size_t bytes, float** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  Workspace& w = g_ws[{dev, s}];
  int rc = grow(s, reinterpret_cast<void**>(&(w.*buf)), &(w.*have), bytes);
  if (rc) return rc;
  *out = w.*buf;
  return SDQ_OK;
}

// The (device, stream) workspace's row-maxima buffer, at least `bytes`.
int rmax_buffer(int dev, hipStream_t s, size_t bytes, float** out) {
  return ws_floats(dev, s, &Workspace::rmax, &Workspace::rmax_bytes, bytes, out);
}

int check_weight(const sdq_weight* w, int64_t K) {
  if (!w) return set_error(SDQ_ERR_INVALID, "null weight handle");
  if (K != w->K)
    return set_error(SDQ_ERR_INVALID, "K mismatch: activations have K=" + std::to_string(K) +
                                          ", weight has K=" + std::to_string(w->K));
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if (dev != w->device)
    return set_error(SDQ_ERR_INVALID, "weight lives on device " + std::to_string(w->device) +
                                          ", current device is " + std::to_string(dev));
  return SDQ_OK;
}

// Size limits of the GEMM kernels, whose in-tile offsets, panel sizes and
// tile counters are 32-bit: a weight of at most 2^20 outputs and 2^22 inputs,
// at most 2^30 rows per call, and fewer than 2^40 output values.
constexpr int64_t kMaxWeightN = int64_t(1) << 20;
constexpr int64_t kMaxWeightK = int64_t(1) << 22;
constexpr int64_t kMaxRows = int64_t(1) << 30;
constexpr int64_t kMaxOutputs = int64_t(1) << 40;

int check_rows(int64_t M, int64_t N, const std::string& tag) {
  if (M > kMaxRows) return set_error(SDQ_ERR_INVALID, tag + "M too large (at most 2^30 rows)");
  if (M * N >= kMaxOutputs)
    return set_error(SDQ_ERR_INVALID, tag + "output too large (M*N must stay under 2^40)");
  return SDQ_OK;
}

int alloc_weight(int dev, int64_t N, int64_t K, sdq_weight** out) {
  if (N < 0 || K < 0) return set_error(SDQ_ERR_INVALID, "negative weight dims");
  if (N > kMaxWeightN || K > kMaxWeightK)
    return set_error(SDQ_ERR_INVALID, "weight too large: N at most 2^20, K at most 2^22 (N=" +
                                          std::to_string(N) + ", K=" + std::to_string(K) + ")");
  const int64_t Np = round_up(N < 1 ? 1 : N, kRowAlign);
  const int64_t KFp = kfrags_padded(K);
  const int64_t bytes = (Np / kFragRows) * KFp * kFragBytes;
  if (bytes >= (int64_t(1) << 40)) return set_error(SDQ_ERR_INVALID, "weight too large");
  sdq_weight* w = new (std::nothrow) sdq_weight{dev, N, K, Np, KFp, nullptr, nullptr};
  if (!w) return set_error(SDQ_ERR_NOMEM, "host allocation failed");
  hipError_t e = hipMalloc(&w->frags, (size_t)bytes);
  if (e == hipSuccess) e = hipMalloc(&w->scale, (size_t)Np * sizeof(float));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (w->frags) (void)hipFree(w->frags);
    delete w;
    return set_error(SDQ_ERR_NOMEM, "weight allocation of " + std::to_string(bytes) +
                                        " bytes failed");
  }
  *out = w;
  return SDQ_OK;
}

EpiArgs make_epi(const sdq_epilogue* epi, int64_t K) {
  EpiArgs e{};
  e.kind = epi ? epi->kind : SDQ_EPI_NONE;
  e.gate_fma = epi ? epi->gate_fma : 1;
  e.kzero = K == 0 ? 1 : 0;
  e.bias = epi ? epi->bias : nullptr;
  e.gate = epi ? epi->gate : nullptr;
  e.resid = epi ? epi->resid : nullptr;
  return e;
}

int validate_epi(const sdq_epilogue* epi) {
  if (!epi) return SDQ_OK;
  switch (epi->kind) {
    case SDQ_EPI_NONE:
    case SDQ_EPI_GELU:
    case SDQ_EPI_ACC:
      return SDQ_OK;
    case SDQ_EPI_GATED:
      if (!epi->gate || !epi->resid)
        return set_error(SDQ_ERR_INVALID, "GATED epilogue needs gate and resid");
      return SDQ_OK;
    case SDQ_EPI_RESID:
      if (!epi->resid) return set_error(SDQ_ERR_INVALID, "RESID epilogue needs resid");
      return SDQ_OK;
    default:
      return set_error(SDQ_ERR_INVALID, "unknown epilogue kind " + std::to_string(epi->kind));
  }
}

}  // namespace

int set_error(int code, const std::string& msg) {
  t_err = msg;
  return code;
}

int hip_error(hipError_t e, const char* what) {
  t_err = std::string(what) + ": " + hipGetErrorString(e);
  return e == hipErrorOutOfMemory ? SDQ_ERR_NOMEM : SDQ_ERR_HIP;
}

// Row maxima handed from a GELU GEMM's epilogue to the next quantizer:
// p[row * stride + c], c < chunks (chunks = 0: not written).
struct RowMax {
  float* p = nullptr;
  int stride = 0;
  int chunks = 0;
};

// Norm + modulation folded into the activation quantizer: the GEMM's rows
// are mod_rows(layernorm(A, eps), shift, scale).
struct LnMod {
  const float* shift;
  const float* scale;
  float eps;
};

// Core device-pointer path shared by the entry points. `pre` (nullable):
// A's row maxima are known; `rmax_out` (nullable, GELU): write Y's; `lnmod`
// (nullable): quantize mod_rows(layernorm(A)) instead of A.
// `fixed` (nullable): the no-alloc mode, all scratch carved from this
// device's static scratch array instead of the grown workspace (nothing is
// allocated; no profiling events are made).
int qlinear_device(const sdq_weight* w, const float* A, int64_t M, int64_t K,
                   const sdq_epilogue* epi, void* Y, hipStream_t s, const RowMax* pre = nullptr,
                   RowMax* rmax_out = nullptr, const LnMod* lnmod = nullptr,
                   char* fixed = nullptr) {
  if (fixed && (pre || rmax_out || lnmod))
    return set_error(SDQ_ERR_INVALID, "no-alloc mode covers the plain qlinear only");
  const bool prof = t_prof && !fixed;
  int rc = check_weight(w, K);
  if (rc) return rc;
  if ((rc = validate_epi(epi))) return rc;
  if (M < 0) return set_error(SDQ_ERR_INVALID, "negative M");
  if (M == 0 || w->N == 0) return SDQ_OK;
  if (!A && K > 0) return set_error(SDQ_ERR_INVALID, "null A");
  if (!Y) return set_error(SDQ_ERR_INVALID, "null Y");
  if ((rc = ensure_device(w->device))) return rc;
  const int64_t N = w->N;
  if ((rc = check_rows(M, N, ""))) return rc;

  const int cfg = choose_gemm_cfg(M, N, w->KFp, epi ? epi->kind : SDQ_EPI_NONE,
                                  g_dev[w->device].cu_count);
  if (lnmod && (!lnmod->shift || !lnmod->scale || K == 0))
    return set_error(SDQ_ERR_INVALID, "layernorm+modulation needs shift, scale and K > 0");
  if (!lnmod && cfg == kCfgSkinny && qin_fits(M, K, w->KFp) && !std::getenv("SDQ_NO_QIN")) {
    // a few rows: the GEMM quantizes them itself (SDQ_NO_QIN: the two-launch
    // path, for comparisons)
    const EpiArgs ea = make_epi(epi, K);
    int vec = (N % 4 == 0) && aligned16(Y);
    if (ea.bias) vec = vec && aligned16(ea.bias);
    if (ea.gate) vec = vec && aligned16(ea.gate);
    if (ea.resid) vec = vec && aligned16(ea.resid);
    if (rmax_out) rmax_out->chunks = 0;
    hipEvent_t p0 = prof ? prof_mark(s) : nullptr;
    hipError_t e = launch_qgemm_qin(w->frags, w->scale, A, M, K, N, w->KFp, ea, Y, vec, s);
    if (e != hipSuccess) {
      drop_events({p0});
      return hip_error(e, "qgemm launch");
    }
    if (prof) {
      hipEvent_t p1 = prof_mark(s);
      if (p0 && p1) {
        t_recs.push_back({"qgemm_skinny_qin", p0, p1});
      } else {
        for (hipEvent_t ev : {p0, p1})
          if (ev) (void)hipEventDestroy(ev);
      }
    }
    return SDQ_OK;
  }
  const int64_t Mp = round_up(M, gemm_cfg_bm(cfg));
  const size_t at_bytes = (size_t)(Mp / kFragRows) * (size_t)w->KFp * kFragBytes;
  const size_t col_cap = (size_t)(w->Np + kColPad);
  Workspace* ws = nullptr;
  const int splitk = choose_splitk(cfg, M, N, w->KFp, g_dev[w->device].cu_count);
  const size_t part_bytes = splitk > 1 ? (size_t)splitk * (size_t)M * (size_t)N * 4 : 0;
  const int cu_count = g_dev[w->device].cu_count;
  const size_t pmax_bytes = (size_t)act_quant_pmax_floats(Mp, w->KFp, cu_count) * sizeof(float);
  Workspace fixed_ws;
  if (fixed) {
    // Every region is rewritten by this call's kernels before it is read
    // (the quantizer writes all Mp rows of fragments and the padded column
    // copies; split-K items write their whole slices; the pmax kernel every
    // chunk it hands on), so nothing needs clearing between calls.
    size_t off = 0;
    auto take = [&](size_t bytes) {
      char* p = fixed + off;
      off += (size_t)round_up((int64_t)bytes, 256);
      return p;
    };
    fixed_ws.at = reinterpret_cast<int8_t*>(take(at_bytes));
    fixed_ws.as = reinterpret_cast<float*>(take((size_t)Mp * sizeof(float)));
    fixed_ws.cols = reinterpret_cast<float*>(take(col_cap * 2 * sizeof(float)));
    fixed_ws.col_cap = col_cap;
    fixed_ws.sink = reinterpret_cast<float*>(take(4096));
    if (part_bytes) fixed_ws.part = reinterpret_cast<int*>(take(part_bytes));
    if (pmax_bytes) fixed_ws.pmax = reinterpret_cast<float*>(take(pmax_bytes));
    if (off > (size_t)SDQ_NOALLOC_SCRATCH_BYTES)
      return set_error(SDQ_ERR_INVALID,
                       "sdq_qlinear_noalloc: M=" + std::to_string(M) + ", K=" + std::to_string(K) +
                           ", N=" + std::to_string(N) + " needs " + std::to_string(off) +
                           " bytes of scratch; the no-alloc entry point has " +
                           std::to_string((size_t)SDQ_NOALLOC_SCRATCH_BYTES));
    ws = &fixed_ws;
  } else if ((rc = workspace(w->device, s, at_bytes, (size_t)Mp * sizeof(float), col_cap,
                             part_bytes, pmax_bytes, &ws))) {
    return rc;
  }
  EpiArgs ea = make_epi(epi, K);
  if (rmax_out) {
    ea.rmax = rmax_out->p;
    ea.rmax_stride = rmax_out->stride;
    rmax_out->chunks = 0;
  }
  const bool premax = !lnmod && pre && pre->chunks > 0;
  if (lnmod) {
    std::lock_guard<std::mutex> lk(g_mu);
    if ((rc = grow(s, reinterpret_cast<void**>(&ws->st), &ws->st_bytes,
                   (size_t)M * sizeof(float2))))
      return rc;
  }
  ColCopy cc{};
  cc.bias = ea.bias;
  cc.gate = ea.gate;
  cc.bias_pad = ea.bias ? ws->cols : nullptr;
  cc.gate_pad = ea.gate ? ws->cols + ws->col_cap : nullptr;
  cc.N = N;
  cc.CP = (int64_t)col_cap;

  hipEvent_t p0 = prof ? prof_mark(s) : nullptr;
  hipError_t e =
      lnmod ? launch_act_quant_frags_lnmod(A, M, K, Mp, w->KFp, ws->at, ws->as, cc, lnmod->shift,
                                           lnmod->scale, lnmod->eps, ws->st, s)
      : premax ? launch_act_quant_frags_premax(A, M, K, Mp, w->KFp, ws->at, ws->as, cc, pre->p,
                                               pre->chunks, pre->stride, cu_count, s)
               : launch_act_quant_frags(A, M, K, Mp, w->KFp, ws->at, ws->as, cc,
                                        pmax_bytes ? ws->pmax : nullptr, cu_count, s);
  if (e != hipSuccess) {
    drop_events({p0});
    return hip_error(e, "act_quant launch");
  }
  hipEvent_t p1 = prof ? prof_mark(s) : nullptr;
  int vec = (N % 4 == 0) && aligned16(Y);
  if (ea.bias) vec = vec && aligned16(ea.bias);
  if (ea.gate) vec = vec && aligned16(ea.gate);
  if (ea.resid) vec = vec && aligned16(ea.resid);
  int tail = 0;
  hipEvent_t pmid = nullptr;
  if (prof && hipEventCreate(&pmid) != hipSuccess) pmid = nullptr;
  GemmAux aux{cc.bias_pad, cc.gate_pad, ws->sink, g_dev[w->device].cu_count, splitk,
              splitk > 1 ? ws->part : nullptr, rmax_out ? &rmax_out->chunks : nullptr, &tail,
              pmid};
  e = launch_qgemm(cfg, w->frags, w->scale, ws->at, ws->as, M, N, w->KFp, ea, Y, vec, aux, s);
  if (e != hipSuccess) {
    drop_events({p0, p1, pmid});
    return hip_error(e, "qgemm launch");
  }
  if (prof) {
    hipEvent_t p2 = prof_mark(s);
    if (p0 && p1 && p2 && (!tail || pmid)) {
      t_recs.push_back({lnmod ? "ln_mod_quant" : premax ? "act_quant_premax" : "act_quant", p0, p1});
      const std::string g = std::string("qgemm_") + gemm_cfg_name(cfg) + (splitk > 1 ? "_splitk" : "");
      if (tail) {
        // the 256x256 launch over the full rounds' rows, then the 128x128
        // launch over the remaining rows: one record each
        t_recs.push_back({g, p1, pmid});
        t_recs.push_back({"qgemm_tail128", pmid, p2});
        pmid = nullptr;
      } else {
        t_recs.push_back({g, p1, p2});
      }
    } else {
      for (hipEvent_t ev : {p0, p1, p2})
        if (ev) (void)hipEventDestroy(ev);
    }
  }
  if (pmid) (void)hipEventDestroy(pmid);
  return SDQ_OK;
}

// sdq_ffn / sdq_ffn_lnmod: fc1 (GELU, row maxima out) then fc2 (gated, row
// maxima in); lnmod folds the FFN's norm + modulation into fc1's quantizer.
int ffn_device(const sdq_weight* fc1, const float* b1, const sdq_weight* fc2, const float* b2,
               const float* h, int64_t M, const float* gate, int gate_fma, float* hid, float* x,
               hipStream_t s, const LnMod* lnmod) {
  if (!fc1 || !fc2) return set_error(SDQ_ERR_INVALID, "null weight handle");
  if (fc2->K != fc1->N || fc2->N != fc1->K)
    return set_error(SDQ_ERR_INVALID,
                     "ffn: fc1 is [" + std::to_string(fc1->N) + "," + std::to_string(fc1->K) +
                         "], fc2 is [" + std::to_string(fc2->N) + "," + std::to_string(fc2->K) +
                         "]; need fc1 [F,D] and fc2 [D,F]");
  if (fc1->device != fc2->device)
    return set_error(SDQ_ERR_INVALID, "ffn: fc1 and fc2 are on different devices");
  if (!gate || !hid || !x) return set_error(SDQ_ERR_INVALID, "ffn: null gate, hid or x");
  if (M < 0) return set_error(SDQ_ERR_INVALID, "negative M");
  if (M == 0) return SDQ_OK;
  int rc = ensure_device(fc1->device);
  if (rc) return rc;
  // fc1's GELU epilogue writes hid's row maxima (either persistent tile
  // config: two wave columns per tile) for fc2's quantizer.
  RowMax rm;
  rm.stride = (int)round_up(std::max(gemm_rmax_chunks(kCfg128x128, fc1->N),
                                     gemm_rmax_chunks(kCfg256x256, fc1->N)),
                            4);
  if ((rc = rmax_buffer(fc1->device, s, (size_t)M * rm.stride * sizeof(float), &rm.p))) return rc;
  sdq_epilogue e1{SDQ_EPI_GELU, 1, b1, nullptr, nullptr};
  if ((rc = qlinear_device(fc1, h, M, fc1->K, &e1, hid, s, nullptr, &rm, lnmod))) return rc;
  sdq_epilogue e2{SDQ_EPI_GATED, gate_fma, b2, gate, x};
  return qlinear_device(fc2, hid, M, fc2->K, &e2, x, s, &rm, nullptr);
}

}  // namespace sdq

using namespace sdq;

extern "C" {

const char* sdq_last_error(void) { return t_err.c_str(); }

#ifndef SDQ_SRC_HASH
#define SDQ_SRC_HASH "unknown"
#endif
const char* sdq_version(void) { return "sdq 0.2 gfx950 src:" SDQ_SRC_HASH; }

int sdq_init(int device) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_error(e, "hipGetDeviceCount");
  if (device < 0 || device >= n || device >= kMaxDev)
    return set_error(SDQ_ERR_NODEV, "no device " + std::to_string(device) + " (" +
                                        std::to_string(n) + " visible)");
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_error(e, "hipSetDevice");
  return ensure_device(device);
}

int sdq_device_info_get(sdq_device_info* out) {
  if (!out) return set_error(SDQ_ERR_INVALID, "null out");
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  const hipDeviceProp_t& p = g_dev[dev].prop;
  out->device = dev;
  out->cu_count = p.multiProcessorCount;
  out->max_clock_khz = p.clockRate;
  out->mem_clock_khz = p.memoryClockRate;
  out->total_mem = (int64_t)p.totalGlobalMem;
  std::snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
  return SDQ_OK;
}

int sdq_weight_upload(const int8_t* q, const float* scale, int64_t N, int64_t K, void* stream,
                      sdq_weight** out) {
  if (!out) return set_error(SDQ_ERR_INVALID, "null out");
  *out = nullptr;
  if (N < 0 || K < 0) return set_error(SDQ_ERR_INVALID, "negative weight dims");
  if ((N * K > 0 && !q) || (N > 0 && !scale)) return set_error(SDQ_ERR_INVALID, "null weight data");
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  sdq_weight* w = nullptr;
  if ((rc = alloc_weight(dev, N, K, &w))) return rc;
  // Stage the .sdcpp blob as it is on disk (int8 rows, then the scales,
  // which may be unaligned in the source) into one device buffer.
  const size_t qbytes = (size_t)(N * K);
  const size_t soff = (size_t)round_up((int64_t)qbytes, 256);
  const size_t sbytes = (size_t)N * 4;
  void* stage = nullptr;
  hipError_t e = hipMalloc(&stage, soff + sbytes + 16);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    sdq_weight_free(w);
    return set_error(SDQ_ERR_NOMEM, "staging allocation failed");
  }
  char* st = static_cast<char*>(stage);
  if (qbytes) e = hipMemcpyAsync(st, q, qbytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess && sbytes) e = hipMemcpyAsync(st + soff, scale, sbytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess)
    e = launch_repack_weight(reinterpret_cast<int8_t*>(st), reinterpret_cast<float*>(st + soff), N,
                             K, w->Np, w->KFp, w->frags, w->scale, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  (void)hipFree(stage);
  if (e != hipSuccess) {
    sdq_weight_free(w);
    return hip_error(e, "weight upload");
  }
  *out = w;
  return SDQ_OK;
}

namespace {

// memcpy split over up to `threads` host threads (page-cache or mmap reads
// run faster in parallel).
void par_memcpy(char* dst, const char* src, size_t bytes, int threads) {
  constexpr size_t kMinPerThread = size_t(4) << 20;
  const int t = (int)std::min<size_t>((size_t)threads, std::max<size_t>(1, bytes / kMinPerThread));
  if (t <= 1) {
    std::memcpy(dst, src, bytes);
    return;
  }
  std::vector<std::thread> pool;
  const size_t chunk = (bytes + t - 1) / t;
  for (int i = 0; i < t; i++) {
    const size_t a = (size_t)i * chunk, b = std::min(bytes, a + chunk);
    if (a < b) pool.emplace_back([=] { std::memcpy(dst + a, src + a, b - a); });
  }
  for (auto& th : pool) th.join();
}

}  // namespace

}  // extern "C"

namespace {

// Streams n weights (weight i: N[i] x K[i] int8 rows + N[i] scales) to the
// device through a ring of pinned staging slots: fill(i, slot, soff) writes
// weight i's int8 rows at slot[0..) and its scales at slot[soff..) on the
// host (several threads), the H2D copy runs on a copy stream, and the GPU
// repack of the previous weight runs on `s` meanwhile. On error no handle is
// returned.
template <class Fill>
int upload_ring(int dev, const std::vector<int64_t>& Ns, const std::vector<int64_t>& Ks, Fill fill,
                hipStream_t s, sdq_weight** out) {
  const int n = (int)Ns.size();
  size_t slot = 0;
  for (int i = 0; i < n; i++)
    slot = std::max(slot, (size_t)round_up(Ns[i] * Ks[i], 256) + (size_t)Ns[i] * 4 + 16);
  constexpr int kSlots = 3;
  const int nslots = std::min(n, kSlots);
  int rc = SDQ_OK;
  hipStream_t cs = nullptr;
  std::vector<char*> pin(nslots, nullptr), dst(nslots, nullptr);
  std::vector<hipEvent_t> copied(nslots, nullptr), repacked(nslots, nullptr);
  hipError_t e = hipStreamCreateWithFlags(&cs, hipStreamNonBlocking);
  for (int k = 0; k < nslots && e == hipSuccess; k++) {
    e = hipHostMalloc(reinterpret_cast<void**>(&pin[k]), slot, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&dst[k]), slot);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&copied[k], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&repacked[k], hipEventDisableTiming);
  }
  for (int i = 0; i < n && e == hipSuccess && rc == SDQ_OK; i++) {
    const int k = i % nslots;
    const int64_t N = Ns[i], K = Ks[i];
    const size_t soff = (size_t)round_up(N * K, 256);
    if ((rc = alloc_weight(dev, N, K, &out[i]))) break;
    // the pinned slot is free once its previous H2D copy has finished
    if (i >= nslots && (e = hipEventSynchronize(copied[k])) != hipSuccess) break;
    if ((rc = fill(i, pin[k], soff))) break;
    // the device slot is free once the repack that read it has run
    if (i >= nslots && (e = hipStreamWaitEvent(cs, repacked[k], 0)) != hipSuccess) break;
    if ((e = hipMemcpyAsync(dst[k], pin[k], soff + (size_t)N * 4, hipMemcpyHostToDevice, cs)) !=
        hipSuccess)
      break;
    if ((e = hipEventRecord(copied[k], cs)) != hipSuccess) break;
    if ((e = hipStreamWaitEvent(s, copied[k], 0)) != hipSuccess) break;
    e = launch_repack_weight(reinterpret_cast<int8_t*>(dst[k]), reinterpret_cast<float*>(dst[k] + soff),
                             N, K, out[i]->Np, out[i]->KFp, out[i]->frags, out[i]->scale, s);
    if (e == hipSuccess) e = hipEventRecord(repacked[k], s);
  }
  if (e == hipSuccess && rc == SDQ_OK) e = hipStreamSynchronize(s);
  if (cs) (void)hipStreamSynchronize(cs);
  if (s) (void)hipStreamSynchronize(s);
  for (int k = 0; k < nslots; k++) {
    if (pin[k]) (void)hipHostFree(pin[k]);
    if (dst[k]) (void)hipFree(dst[k]);
    if (copied[k]) (void)hipEventDestroy(copied[k]);
    if (repacked[k]) (void)hipEventDestroy(repacked[k]);
  }
  if (cs) (void)hipStreamDestroy(cs);
  if (e != hipSuccess && rc == SDQ_OK) rc = hip_error(e, "batch weight upload");
  if (rc != SDQ_OK) {
    const std::string msg = t_err;
    for (int i = 0; i < n; i++) {
      if (out[i]) sdq_weight_free(out[i]);
      out[i] = nullptr;
    }
    t_err = msg;
  }
  return rc;
}

int upload_threads() {
  return (int)std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
}

// One file range to read into host memory.
struct ReadSpan {
  char* dst;
  uint64_t off;
  size_t bytes;
};

// Reads every span, cut into chunks of at most kChunk bytes spread over up to
// `threads` threads: large sequential reads with enough of them in flight for
// a page cache or an NVMe queue. Returns false on a short read or an I/O
// error.
bool read_spans(int fd, const std::vector<ReadSpan>& spans, int threads) {
  constexpr size_t kChunk = size_t(4) << 20;
  std::vector<ReadSpan> chunks;
  for (const ReadSpan& s : spans)
    for (size_t a = 0; a < s.bytes; a += kChunk)
      chunks.push_back({s.dst + a, s.off + a, std::min(kChunk, s.bytes - a)});
  auto one = [fd](const ReadSpan& c) {
    char* d = c.dst;
    uint64_t o = c.off;
    size_t b = c.bytes;
    while (b) {
      const ssize_t got = ::pread(fd, d, b, (off_t)o);
      if (got < 0 && errno == EINTR) continue;
      if (got <= 0) return false;
      d += got;
      o += (uint64_t)got;
      b -= (size_t)got;
    }
    return true;
  };
  const int t = (int)std::min<size_t>((size_t)std::max(threads, 1), chunks.size());
  if (t <= 1) {
    for (const ReadSpan& c : chunks)
      if (!one(c)) return false;
    return true;
  }
  std::atomic<size_t> next{0};
  std::atomic<bool> ok{true};
  std::vector<std::thread> pool;
  for (int i = 0; i < t; i++)
    pool.emplace_back([&] {
      for (size_t j; ok && (j = next.fetch_add(1)) < chunks.size();)
        if (!one(chunks[j])) ok = false;
    });
  for (auto& th : pool) th.join();
  return ok;
}

}  // namespace

namespace {

// sdq_qlinear_host's staging, per host thread and device, grown and never
// shrunk (held until the process ends): a device block for the call's
// arrays, a stream of its own, and two pinned host buffers through which
// host arrays move in chunks (the copy of one chunk into pinned memory
// overlaps the DMA of the previous one).
constexpr size_t kHostBounce = size_t(16) << 20;  // bytes per pinned buffer
struct HostStage {
  hipStream_t stream = nullptr;
  char* dbuf = nullptr;
  size_t dbytes = 0;
  char* pin[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
};
thread_local HostStage t_host_stage[kMaxDev];

int host_stage_ready(HostStage& hs) {
  hipError_t e = hipSuccess;
  if (!hs.stream) {
    e = hipStreamCreateWithFlags(&hs.stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      hs.stream = nullptr;
      return hip_error(e, "hipStreamCreate (host calls)");
    }
  }
  for (int i = 0; i < 2; i++) {
    if (!hs.pin[i]) {
      void* p = nullptr;
      e = hipHostMalloc(&p, kHostBounce, hipHostMallocDefault);
      if (e != hipSuccess) return hip_error(e, "hipHostMalloc (host-call bounce)");
      hs.pin[i] = static_cast<char*>(p);
    }
    if (!hs.done[i]) {
      e = hipEventCreateWithFlags(&hs.done[i], hipEventDisableTiming);
      if (e != hipSuccess) {
        hs.done[i] = nullptr;
        return hip_error(e, "hipEventCreate (host calls)");
      }
    }
  }
  return SDQ_OK;
}

// Host -> device through the pinned buffers. A buffer is refilled only
// after the DMA that read it finished.
int host_stage_h2d(HostStage& hs, char* dst, const void* src, size_t bytes) {
  const char* p = static_cast<const char*>(src);
  for (size_t off = 0, c = 0; off < bytes; off += kHostBounce, c++) {
    const size_t len = bytes - off < kHostBounce ? bytes - off : kHostBounce;
    const int b = (int)(c & 1);
    hipError_t e = hipEventSynchronize(hs.done[b]);
    if (e == hipSuccess) {
      std::memcpy(hs.pin[b], p + off, len);
      e = hipMemcpyAsync(dst + off, hs.pin[b], len, hipMemcpyHostToDevice, hs.stream);
    }
    if (e == hipSuccess) e = hipEventRecord(hs.done[b], hs.stream);
    if (e != hipSuccess) return hip_error(e, "host-call H2D");
  }
  return SDQ_OK;
}

// Device -> host through the pinned buffers: chunk c's DMA is queued before
// chunk c-1 is copied out of its pinned buffer.
int host_stage_d2h(HostStage& hs, void* dst, const char* src, size_t bytes) {
  char* q = static_cast<char*>(dst);
  size_t prev_off = 0, prev_len = 0;
  int prev_b = -1;
  auto drain = [&]() {
    if (prev_b < 0) return hipSuccess;
    hipError_t e = hipEventSynchronize(hs.done[prev_b]);
    if (e == hipSuccess) std::memcpy(q + prev_off, hs.pin[prev_b], prev_len);
    prev_b = -1;
    return e;
  };
  for (size_t off = 0, c = 0; off < bytes; off += kHostBounce, c++) {
    const size_t len = bytes - off < kHostBounce ? bytes - off : kHostBounce;
    const int b = (int)(c & 1);
    // buffer b last held chunk c-2, copied out when chunk c-1 was queued
    hipError_t e = hipMemcpyAsync(hs.pin[b], src + off, len, hipMemcpyDeviceToHost, hs.stream);
    if (e == hipSuccess) e = hipEventRecord(hs.done[b], hs.stream);
    if (e == hipSuccess) e = drain();
    if (e != hipSuccess) return hip_error(e, "host-call D2H");
    prev_off = off;
    prev_len = len;
    prev_b = b;
  }
  const hipError_t e = drain();
  if (e != hipSuccess) return hip_error(e, "host-call D2H");
  return SDQ_OK;
}

// Whether item `it` takes sdq_qlinear_group's shared launches: the plain
// quantizer's single-kernel form and the 128x128 persistent GEMM without
// split-K, the path sdq_qlinear itself would take for it.
bool groupable(const sdq_group_item& it, int cu_count) {
  const sdq_weight* w = it.w;
  const int kind = it.epi.kind;
  if (kind != SDQ_EPI_NONE && kind != SDQ_EPI_GELU && kind != SDQ_EPI_GATED &&
      kind != SDQ_EPI_RESID)
    return false;
  if (w->K == 0 || it.M > (int64_t(1) << 30)) return false;
  const int64_t N = w->N;
  if (choose_gemm_cfg(it.M, N, w->KFp, kind, cu_count) != kCfg128x128) return false;
  if (choose_splitk(kCfg128x128, it.M, N, w->KFp, cu_count) != 1) return false;
  const int64_t Mp = round_up(it.M, gemm_cfg_bm(kCfg128x128));
  if (act_quant_pmax_floats(Mp, w->KFp, cu_count) != 0) return false;
  if (N % 4 != 0 || !aligned16(it.Y)) return false;
  if (it.epi.bias && !aligned16(it.epi.bias)) return false;
  if (it.epi.gate && !aligned16(it.epi.gate)) return false;
  if (it.epi.resid && !aligned16(it.epi.resid)) return false;
  return w->KFp * 1024 * 8 <= 0x7FFFFFFF && N * 4 * 256 <= 0x7FFFFFF0;
}

// Whether a Linear of sdq_qlinear_stack can run from an input quantized by
// the stack's shared launch: one persistent launch of the tile config
// qlinear_device would choose, without split-K, whose quantizer would be the
// single-kernel form (the shared launch runs that form's per-unit code),
// with the vector epilogue. *cfg: that tile config.
bool stackable(const sdq_weight* w, int64_t M, int kind, const void* Y, const float* bias,
               const float* gate, const float* resid, int cu_count, int* cfg) {
  if (kind != SDQ_EPI_NONE && kind != SDQ_EPI_GELU && kind != SDQ_EPI_GATED &&
      kind != SDQ_EPI_RESID)
    return false;
  const int64_t N = w->N;
  if (w->K == 0 || M <= 0 || M > (int64_t(1) << 30) || N % 4 != 0) return false;
  const int c = choose_gemm_cfg(M, N, w->KFp, kind, cu_count);
  if (c != kCfg128x128 && c != kCfg256x256) return false;
  if (choose_splitk(c, M, N, w->KFp, cu_count) != 1) return false;
  if (act_quant_pmax_floats(round_up(M, gemm_cfg_bm(c)), w->KFp, cu_count) != 0) return false;
  if (!aligned16(Y) || (bias && !aligned16(bias)) || (gate && !aligned16(gate)) ||
      (resid && !aligned16(resid)))
    return false;
  *cfg = c;
  return w->KFp * 1024 * 8 <= 0x7FFFFFFF && N * 4 * 256 <= 0x7FFFFFF0;
}

// Items that may share one GEMM launch: the same k-fragments (the launch
// reads each problem's epilogue form from its table).
bool same_group(const sdq_group_item& a, const sdq_group_item& b) {
  return a.w->KFp == b.w->KFp;
}

}  // namespace

extern "C" {

int sdq_weight_upload_batch(const sdq_weight_src* src, int n, void* stream, sdq_weight** out) {
  if (!out || (n > 0 && !src)) return set_error(SDQ_ERR_INVALID, "null src or out");
  if (n < 0) return set_error(SDQ_ERR_INVALID, "negative count");
  for (int i = 0; i < n; i++) out[i] = nullptr;
  if (n == 0) return SDQ_OK;
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  std::vector<int64_t> Ns(n), Ks(n);
  for (int i = 0; i < n; i++) {
    const sdq_weight_src& w = src[i];
    if (w.nparts < 1 || w.nparts > 4 || w.K < 0)
      return set_error(SDQ_ERR_INVALID, "weight source " + std::to_string(i) + ": bad parts or K");
    int64_t N = 0;
    for (int p = 0; p < w.nparts; p++) {
      if (w.rows[p] < 0 || (w.rows[p] * w.K > 0 && !w.q[p]) || (w.rows[p] > 0 && !w.scale[p]))
        return set_error(SDQ_ERR_INVALID, "weight source " + std::to_string(i) + ": null part");
      N += w.rows[p];
    }
    Ns[i] = N;
    Ks[i] = w.K;
  }
  const int threads = upload_threads();
  auto fill = [&](int i, char* pin, size_t soff) {
    const sdq_weight_src& w = src[i];
    size_t r = 0;
    for (int p = 0; p < w.nparts; p++) {
      par_memcpy(pin + r * (size_t)w.K, reinterpret_cast<const char*>(w.q[p]),
                 (size_t)(w.rows[p] * w.K), threads);
      std::memcpy(pin + soff + r * 4, w.scale[p], (size_t)w.rows[p] * 4);
      r += (size_t)w.rows[p];
    }
    return SDQ_OK;
  };
  return upload_ring(dev, Ns, Ks, fill, static_cast<hipStream_t>(stream), out);
}

int sdq_weight_upload_file(const char* path, const sdq_weight_fsrc* src, int n, void* stream,
                           sdq_weight** out) {
  if (!path || !out || (n > 0 && !src)) return set_error(SDQ_ERR_INVALID, "null path, src or out");
  if (n < 0) return set_error(SDQ_ERR_INVALID, "negative count");
  for (int i = 0; i < n; i++) out[i] = nullptr;
  if (n == 0) return SDQ_OK;
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return set_error(SDQ_ERR_NOTFOUND, std::string("cannot open ") + path);
  struct stat st;
  if (::fstat(fd, &st) != 0) {
    ::close(fd);
    return set_error(SDQ_ERR_FORMAT, std::string("cannot stat ") + path);
  }
  const uint64_t size = (uint64_t)st.st_size;
  std::vector<int64_t> Ns(n), Ks(n);
  for (int i = 0; i < n && rc == SDQ_OK; i++) {
    const sdq_weight_fsrc& w = src[i];
    if (w.nparts < 1 || w.nparts > 4 || w.K < 0) {
      rc = set_error(SDQ_ERR_INVALID, "weight source " + std::to_string(i) + ": bad parts or K");
      break;
    }
    int64_t N = 0;
    for (int p = 0; p < w.nparts; p++) {
      const uint64_t qb = (uint64_t)(w.rows[p] * w.K), sb = (uint64_t)w.rows[p] * 4;
      if (w.rows[p] < 0 || w.q_off[p] > size || qb > size - w.q_off[p] ||
          w.scale_off[p] > size || sb > size - w.scale_off[p]) {
        rc = set_error(SDQ_ERR_FORMAT, "weight source " + std::to_string(i) + ": part " +
                                           std::to_string(p) + " lies outside " + path);
        break;
      }
      N += w.rows[p];
    }
    Ns[i] = N;
    Ks[i] = w.K;
  }
  if (rc == SDQ_OK) {
    (void)::posix_fadvise(fd, 0, 0, POSIX_FADV_SEQUENTIAL);
    const int threads = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    // the kernel's read-ahead of a weight's ranges (no wait)
    auto prefetch = [&](int i) {
      if (i >= n) return;
      const sdq_weight_fsrc& w = src[i];
      for (int p = 0; p < w.nparts; p++) {
        (void)::posix_fadvise(fd, (off_t)w.q_off[p], (off_t)(w.rows[p] * w.K), POSIX_FADV_WILLNEED);
        (void)::posix_fadvise(fd, (off_t)w.scale_off[p], (off_t)(w.rows[p] * 4), POSIX_FADV_WILLNEED);
      }
    };
    prefetch(0);
    auto fill = [&](int i, char* pin, size_t soff) {
      prefetch(i + 1);
      const sdq_weight_fsrc& w = src[i];
      std::vector<ReadSpan> spans;
      size_t r = 0;
      for (int p = 0; p < w.nparts; p++) {
        spans.push_back({pin + r * (size_t)w.K, w.q_off[p], (size_t)(w.rows[p] * w.K)});
        spans.push_back({pin + soff + r * 4, w.scale_off[p], (size_t)w.rows[p] * 4});
        r += (size_t)w.rows[p];
      }
      if (!read_spans(fd, spans, threads))
        return set_error(SDQ_ERR_FORMAT, std::string("short read from ") + path);
      return SDQ_OK;
    };
    rc = upload_ring(dev, Ns, Ks, fill, static_cast<hipStream_t>(stream), out);
  }
  ::close(fd);
  return rc;
}

int sdq_weight_upload_device(const int8_t* q_dev, const float* scale_dev, int64_t N, int64_t K,
                             void* stream, sdq_weight** out) {
  if (!out) return set_error(SDQ_ERR_INVALID, "null out");
  *out = nullptr;
  if (N < 0 || K < 0) return set_error(SDQ_ERR_INVALID, "negative weight dims");
  if ((N * K > 0 && !q_dev) || (N > 0 && !scale_dev))
    return set_error(SDQ_ERR_INVALID, "null weight data");
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  sdq_weight* w = nullptr;
  if ((rc = alloc_weight(dev, N, K, &w))) return rc;
  hipError_t e = launch_repack_weight(q_dev, scale_dev, N, K, w->Np, w->KFp, w->frags, w->scale, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    sdq_weight_free(w);
    return hip_error(e, "weight repack");
  }
  *out = w;
  return SDQ_OK;
}

int sdq_weight_free(sdq_weight* w) {
  if (!w) return SDQ_OK;
  if (w->frags) (void)hipFree(w->frags);
  if (w->scale) (void)hipFree(w->scale);
  delete w;
  return SDQ_OK;
}

int sdq_weight_dims(const sdq_weight* w, int64_t* N, int64_t* K) {
  if (!w) return set_error(SDQ_ERR_INVALID, "null weight handle");
  if (N) *N = w->N;
  if (K) *K = w->K;
  return SDQ_OK;
}

int sdq_weight_export_host(const sdq_weight* w, int8_t* q, float* scale) {
  if (!w) return set_error(SDQ_ERR_INVALID, "null weight handle");
  const size_t qbytes = (size_t)(w->N * w->K);
  int8_t* tmp = nullptr;
  hipError_t e = hipSuccess;
  if (qbytes) {
    e = hipMalloc(&tmp, qbytes);
    if (e != hipSuccess) return hip_error(e, "hipMalloc");
    e = launch_unpack_weight(w->frags, w->N, w->K, w->KFp, tmp, nullptr);
    if (e == hipSuccess) e = hipMemcpy(q, tmp, qbytes, hipMemcpyDeviceToHost);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_error(e, "weight export");
  }
  if (scale && w->N) {
    e = hipMemcpy(scale, w->scale, (size_t)w->N * 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_error(e, "scale export");
  }
  return SDQ_OK;
}

int sdq_qlinear(const sdq_weight* w, const float* A, int64_t M, int64_t K, const sdq_epilogue* epi,
                void* Y, void* stream) {
  return qlinear_device(w, A, M, K, epi, Y, static_cast<hipStream_t>(stream));
}


int sdq_qlinear_group(const sdq_group_item* items, int n, void* stream) {
  if (n < 0 || n > SDQ_MAX_GROUP) return set_error(SDQ_ERR_INVALID, "group: n must be 0..16");
  if (n > 0 && !items) return set_error(SDQ_ERR_INVALID, "group: null items");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  // the checks sdq_qlinear makes, for every item before anything runs
  for (int i = 0; i < n; i++) {
    const sdq_group_item& it = items[i];
    if (!it.w) return set_error(SDQ_ERR_INVALID, "group item " + std::to_string(i) + ": null weight");
    if ((rc = check_weight(it.w, it.w->K))) return rc;
    if ((rc = validate_epi(&it.epi))) return rc;
    if (it.M < 0) return set_error(SDQ_ERR_INVALID, "group item " + std::to_string(i) + ": negative M");
    if ((rc = check_rows(it.M, it.w->N, "group item " + std::to_string(i) + ": "))) return rc;
    if (it.M > 0 && it.w->N > 0 && ((!it.A && it.w->K > 0) || !it.Y))
      return set_error(SDQ_ERR_INVALID, "group item " + std::to_string(i) + ": null A or Y");
  }
  // The items run in any order (the shared path quantizes every input before
  // any GEMM), so no item's output may overlap another item's input,
  // residual or output.
  {
    struct Span {
      uintptr_t lo, hi;
    };
    auto span = [](const void* p, int64_t bytes) {
      const uintptr_t a = reinterpret_cast<uintptr_t>(p);
      return Span{a, a + (uintptr_t)(bytes > 0 ? bytes : 0)};
    };
    auto meet = [](Span a, Span b) { return a.lo < a.hi && b.lo < b.hi && a.lo < b.hi && b.lo < a.hi; };
    for (int i = 0; i < n; i++) {
      const sdq_group_item& a = items[i];
      if (a.M == 0 || a.w->N == 0) continue;
      const Span ya = span(a.Y, a.M * a.w->N * 4);
      for (int j = 0; j < n; j++) {
        const sdq_group_item& b = items[j];
        if (j == i || b.M == 0 || b.w->N == 0) continue;
        const bool clash = meet(ya, span(b.A, b.M * b.w->K * 4)) ||
                           meet(ya, span(b.Y, b.M * b.w->N * 4)) ||
                           (b.epi.resid && meet(ya, span(b.epi.resid, b.M * b.w->N * 4)));
        if (clash)
          return set_error(SDQ_ERR_INVALID, "group item " + std::to_string(i) +
                                                ": Y overlaps the input, residual or output of item " +
                                                std::to_string(j));
      }
    }
  }
  if ((rc = ensure_device(dev))) return rc;
  const int cu_count = g_dev[dev].cu_count;
  // items of the shared launches, and the rest
  std::vector<int> shared, single;
  for (int i = 0; i < n; i++) {
    if (items[i].M == 0 || items[i].w->N == 0) continue;
    (groupable(items[i], cu_count) ? shared : single).push_back(i);
  }
  // a lone groupable item gains nothing from the shared launches
  if (shared.size() == 1) {
    single.push_back(shared[0]);
    shared.clear();
  }
  if (!shared.empty()) {
    // scratch: per item its quantized rows, row scales and padded column copies
    struct Carve {
      size_t at, as, cols;
    };
    std::vector<Carve> cv(shared.size());
    size_t off = 0;
    auto take = [&](size_t bytes) {
      const size_t o = off;
      off += (size_t)round_up((int64_t)bytes, 256);
      return o;
    };
    const size_t sink_off = take(4096);
    for (size_t j = 0; j < shared.size(); j++) {
      const sdq_group_item& it = items[shared[j]];
      const int64_t Mp = round_up(it.M, gemm_cfg_bm(kCfg128x128));
      cv[j].at = take((size_t)(Mp / kFragRows) * (size_t)it.w->KFp * kFragBytes);
      cv[j].as = take((size_t)Mp * sizeof(float));
      cv[j].cols = take((size_t)(it.w->Np + kColPad) * 2 * sizeof(float));
    }
    char* base = nullptr;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      Workspace& ws = g_ws[{dev, s}];
      if ((rc = grow(s, reinterpret_cast<void**>(&ws.grp), &ws.grp_bytes, off))) return rc;
      base = ws.grp;
    }
    QuantSegs qs{};
    qs.count = (int)shared.size();
    int64_t units = 0;
    for (size_t j = 0; j < shared.size(); j++) {
      const sdq_group_item& it = items[shared[j]];
      const int64_t Mp = round_up(it.M, gemm_cfg_bm(kCfg128x128));
      const int64_t cap = it.w->Np + kColPad;
      QuantSeg& q = qs.s[j];
      q.A = it.A;
      q.M = it.M;
      q.K = it.w->K;
      q.KFp = it.w->KFp;
      q.vec = (aligned16(it.A) && it.w->K % 4 == 0) ? 1 : 0;
      q.at = reinterpret_cast<int8_t*>(base + cv[j].at);
      q.as = reinterpret_cast<float*>(base + cv[j].as);
      float* cols = reinterpret_cast<float*>(base + cv[j].cols);
      q.cc.bias = it.epi.bias;
      q.cc.gate = it.epi.gate;
      q.cc.bias_pad = it.epi.bias ? cols : nullptr;
      q.cc.gate_pad = it.epi.gate ? cols + cap : nullptr;
      q.cc.N = it.w->N;
      q.cc.CP = cap;
      q.unit0 = units;
      units += Mp / 8;
    }
    qs.total = units;
    hipEvent_t p0 = t_prof ? prof_mark(s) : nullptr;
    hipError_t e = launch_act_quant_segs(qs, s);
    if (e != hipSuccess) {
      drop_events({p0});
      return hip_error(e, "group act_quant launch");
    }
    hipEvent_t p1 = t_prof ? prof_mark(s) : nullptr;
    // one GEMM launch per set of items with the same K (each problem carries
    // its own epilogue form)
    std::vector<bool> done(shared.size(), false);
    for (size_t j = 0; j < shared.size(); j++) {
      if (done[j]) continue;
      GemmGroup g{};
      const sdq_group_item& first = items[shared[j]];
      for (size_t k = j; k < shared.size(); k++) {
        const sdq_group_item& it = items[shared[k]];
        if (done[k] || !same_group(first, it)) continue;
        done[k] = true;
        GemmProblem& p = g.p[g.count++];
        p.wt = it.w->frags;
        p.scale = it.w->scale;
        p.bias = qs.s[k].cc.bias_pad;
        p.gate = qs.s[k].cc.gate_pad;
        p.at = qs.s[k].at;
        p.as = qs.s[k].as;
        p.resid = it.epi.resid;
        p.Y = it.Y;
        p.M = (int)it.M;
        p.N = (int)it.w->N;
        p.kind = it.epi.kind;
        p.gate_fma = it.epi.gate_fma;
      }
      EpiArgs ea = make_epi(&first.epi, first.w->K);
      ea.bias = ea.gate = ea.resid = nullptr;  // per problem, from the table
      e = launch_qgemm_group(g, first.w->KFp, ea, reinterpret_cast<float*>(base + sink_off),
                             cu_count, s);
      if (e != hipSuccess) {
        drop_events({p0, p1});
        return hip_error(e, "group qgemm launch");
      }
    }
    if (t_prof) {
      hipEvent_t p2 = prof_mark(s);
      if (p0 && p1 && p2) {
        t_recs.push_back({"act_quant_group", p0, p1});
        t_recs.push_back({"qgemm_group", p1, p2});
      } else {
        for (hipEvent_t ev : {p0, p1, p2})
          if (ev) (void)hipEventDestroy(ev);
      }
    }
  }
  for (int i : single) {
    const sdq_group_item& it = items[i];
    if ((rc = qlinear_device(it.w, it.A, it.M, it.w->K, &it.epi, it.Y, s))) return rc;
  }
  return SDQ_OK;
}

int sdq_qlinear_stack(const sdq_group_item* items, int n, int ngroup, const sdq_ffn_item* ffn,
                      void* stream) {
  if (n < 0 || n > SDQ_MAX_GROUP) return set_error(SDQ_ERR_INVALID, "stack: n must be 0..16");
  if (ngroup < 0 || ngroup > n) return set_error(SDQ_ERR_INVALID, "stack: need 0 <= ngroup <= n");
  if (n > 0 && !items) return set_error(SDQ_ERR_INVALID, "stack: null items");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  for (int i = 0; i < n; i++) {
    const sdq_group_item& it = items[i];
    const std::string tag = "stack item " + std::to_string(i);
    if (!it.w) return set_error(SDQ_ERR_INVALID, tag + ": null weight");
    if ((rc = check_weight(it.w, it.w->K))) return rc;
    if ((rc = validate_epi(&it.epi))) return rc;
    if (it.M < 0) return set_error(SDQ_ERR_INVALID, tag + ": negative M");
    if ((rc = check_rows(it.M, it.w->N, tag + ": "))) return rc;
    if (it.M > 0 && it.w->N > 0 && ((!it.A && it.w->K > 0) || !it.Y))
      return set_error(SDQ_ERR_INVALID, tag + ": null A or Y");
  }
  const bool has_ffn = ffn && ffn->M != 0;
  if (ffn) {
    if (!ffn->fc1 || !ffn->fc2) return set_error(SDQ_ERR_INVALID, "stack: null FFN weight");
    if ((rc = check_weight(ffn->fc1, ffn->fc1->K)) || (rc = check_weight(ffn->fc2, ffn->fc2->K)))
      return rc;
    if (ffn->fc2->K != ffn->fc1->N || ffn->fc2->N != ffn->fc1->K)
      return set_error(SDQ_ERR_INVALID, "stack: need fc1 [F,D] and fc2 [D,F]");
    if (ffn->M < 0) return set_error(SDQ_ERR_INVALID, "stack: negative FFN M");
    if ((rc = check_rows(ffn->M, ffn->fc1->N, "stack FFN: "))) return rc;
    if (has_ffn && ((!ffn->h && ffn->fc1->K > 0) || !ffn->gate || !ffn->hid || !ffn->x))
      return set_error(SDQ_ERR_INVALID, "stack: null FFN h, gate, hid or x");
  }
  // Every input is quantized before any GEMM runs: no output may overlap
  // one. The first ngroup items run in any order among themselves.
  {
    struct Span {
      uintptr_t lo, hi;
      int who;
    };
    auto span = [](const void* p, int64_t bytes, int who) {
      const uintptr_t a = reinterpret_cast<uintptr_t>(p);
      return Span{a, a + (uintptr_t)(bytes > 0 ? bytes : 0), who};
    };
    auto meet = [](Span a, Span b) { return a.lo < a.hi && b.lo < b.hi && a.lo < b.hi && b.lo < a.hi; };
    std::vector<Span> ins, outs;
    for (int i = 0; i < n; i++) {
      const sdq_group_item& it = items[i];
      if (it.M == 0 || it.w->N == 0) continue;
      ins.push_back(span(it.A, it.M * it.w->K * 4, i));
      outs.push_back(span(it.Y, it.M * it.w->N * 4, i));
    }
    if (has_ffn) {
      const int64_t D = ffn->fc1->K, F = ffn->fc1->N;
      ins.push_back(span(ffn->h, ffn->M * D * 4, n));
      outs.push_back(span(ffn->hid, ffn->M * F * 4, n));
      outs.push_back(span(ffn->x, ffn->M * D * 4, n));
    }
    auto who = [&](int i) { return i == n ? std::string("the FFN") : "item " + std::to_string(i); };
    for (const Span& o : outs)
      for (const Span& a : ins)
        if (meet(o, a))
          return set_error(SDQ_ERR_INVALID, "stack: an output of " + who(o.who) +
                                                " overlaps the input of " + who(a.who) +
                                                " (every input is quantized first)");
    for (int i = 0; i < ngroup; i++) {
      const sdq_group_item& a = items[i];
      if (a.M == 0 || a.w->N == 0) continue;
      const Span ya = span(a.Y, a.M * a.w->N * 4, i);
      for (int j = 0; j < ngroup; j++) {
        const sdq_group_item& b = items[j];
        if (j == i || b.M == 0 || b.w->N == 0) continue;
        if (meet(ya, span(b.Y, b.M * b.w->N * 4, j)) ||
            (b.epi.resid && meet(ya, span(b.epi.resid, b.M * b.w->N * 4, j))))
          return set_error(SDQ_ERR_INVALID, "stack: grouped item " + std::to_string(i) +
                                                " writes the output or residual of item " +
                                                std::to_string(j));
      }
    }
  }
  if ((rc = ensure_device(dev))) return rc;
  const int cu_count = g_dev[dev].cu_count;
  // The shared-launch plan: every input through the segmented quantizer,
  // each GEMM as the launch its own call would make, minus its quantizer.
  std::vector<int> cfgs(n, -1);
  int nseg = 0, cfg1 = -1;
  bool fast = true;
  for (int i = 0; i < n && fast; i++) {
    const sdq_group_item& it = items[i];
    if (it.M == 0 || it.w->N == 0) continue;
    nseg++;
    if (i < ngroup) {
      fast = groupable(it, cu_count);
      cfgs[i] = kCfg128x128;
    } else {
      fast = stackable(it.w, it.M, it.epi.kind, it.Y, it.epi.bias, it.epi.gate, it.epi.resid,
                       cu_count, &cfgs[i]);
    }
  }
  if (has_ffn && fast) {
    nseg++;
    fast = stackable(ffn->fc1, ffn->M, SDQ_EPI_GELU, ffn->hid, ffn->b1, nullptr, nullptr, cu_count,
                     &cfg1);
  }
  if (!fast || nseg < 2 || nseg > kMaxQuantSegs) {
    // the same calls, one after another
    if (ngroup > 0 && (rc = sdq_qlinear_group(items, ngroup, stream))) return rc;
    for (int i = ngroup; i < n; i++) {
      const sdq_group_item& it = items[i];
      if ((rc = qlinear_device(it.w, it.A, it.M, it.w->K, &it.epi, it.Y, s))) return rc;
    }
    if (has_ffn)
      return ffn_device(ffn->fc1, ffn->b1, ffn->fc2, ffn->b2, ffn->h, ffn->M, ffn->gate,
                        ffn->gate_fma, ffn->hid, ffn->x, s, nullptr);
    return SDQ_OK;
  }
  // The first Linear after the group, when it adds into what a grouped
  // Linear adds into (the cross output projection after the self-attention
  // output, both into x: ovi_dit.cpp:187, 251), joins the grouped launch:
  // both write their plain outputs (bias included) to scratch, and one
  // elementwise pass applies the two residual epilogues to the target in
  // their order, the same bits as the two GEMM epilogues one after the other.
  // (SDQ_NO_STACK_FOLD: the separate launch, for comparisons.)
  int fold_g = -1;
  const int fold_s = ngroup;
  if (fast && ngroup < n && !std::getenv("SDQ_NO_STACK_FOLD")) {
    const sdq_group_item& S = items[fold_s];
    auto adds = [](const sdq_group_item& it) {
      return it.M > 0 && it.w->N > 0 && it.epi.resid == it.Y &&
             (it.epi.kind == SDQ_EPI_GATED || it.epi.kind == SDQ_EPI_RESID);
    };
    if (adds(S) && groupable(S, cu_count))
      for (int j = 0; j < ngroup; j++) {
        const sdq_group_item& G = items[j];
        if (G.Y == S.Y && adds(G) && G.M == S.M && G.w->N == S.w->N && same_group(G, S))
          fold_g = j;
      }
  }
  // scratch: per input its quantized rows (padded to its GEMM's tile), row
  // scales and padded column copies
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (size_t)round_up((int64_t)bytes, 256);
    return o;
  };
  const size_t sink_off = take(4096);
  size_t yg_off = 0, ys_off = 0;  // the folded pair's plain outputs
  if (fold_g >= 0) {
    const size_t b = (size_t)(items[fold_s].M * items[fold_s].w->N) * sizeof(float);
    yg_off = take(b);
    ys_off = take(b);
  }
  struct Carve {
    size_t at, as, cols;
    int seg;
  };
  std::vector<Carve> cv(n + 1, Carve{0, 0, 0, -1});
  struct Input {
    const sdq_weight* w;
    const float* A;
    int64_t M;
    int cfg;
    const float* bias;
    const float* gate;
  };
  std::vector<Input> in;
  std::vector<int> owner;  // item index (n: the FFN's fc1) of each segment
  for (int i = 0; i < n; i++) {
    const sdq_group_item& it = items[i];
    if (it.M == 0 || it.w->N == 0) continue;
    in.push_back(Input{it.w, it.A, it.M, cfgs[i], it.epi.bias, it.epi.gate});
    owner.push_back(i);
  }
  if (has_ffn) {
    in.push_back(Input{ffn->fc1, ffn->h, ffn->M, cfg1, ffn->b1, nullptr});
    owner.push_back(n);
  }
  for (size_t j = 0; j < in.size(); j++) {
    const int64_t Mp = round_up(in[j].M, gemm_cfg_bm(in[j].cfg));
    Carve& c = cv[owner[j]];
    c.at = take((size_t)(Mp / kFragRows) * (size_t)in[j].w->KFp * kFragBytes);
    c.as = take((size_t)Mp * sizeof(float));
    c.cols = take((size_t)(in[j].w->Np + kColPad) * 2 * sizeof(float));
    c.seg = (int)j;
  }
  char* base = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    Workspace& ws = g_ws[{dev, s}];
    if ((rc = grow(s, reinterpret_cast<void**>(&ws.grp), &ws.grp_bytes, off))) return rc;
    base = ws.grp;
  }
  float* sink = reinterpret_cast<float*>(base + sink_off);
  QuantSegs qs{};
  qs.count = (int)in.size();
  int64_t units = 0;
  for (size_t j = 0; j < in.size(); j++) {
    const Input& x = in[j];
    const Carve& c = cv[owner[j]];
    const int64_t Mp = round_up(x.M, gemm_cfg_bm(x.cfg));
    const int64_t cap = x.w->Np + kColPad;
    QuantSeg& q = qs.s[j];
    q.A = x.A;
    q.M = x.M;
    q.K = x.w->K;
    q.KFp = x.w->KFp;
    q.vec = (aligned16(x.A) && x.w->K % 4 == 0) ? 1 : 0;
    q.at = reinterpret_cast<int8_t*>(base + c.at);
    q.as = reinterpret_cast<float*>(base + c.as);
    float* cols = reinterpret_cast<float*>(base + c.cols);
    q.cc.bias = x.bias;
    q.cc.gate = x.gate;
    q.cc.bias_pad = x.bias ? cols : nullptr;
    q.cc.gate_pad = x.gate ? cols + cap : nullptr;
    q.cc.N = x.w->N;
    q.cc.CP = cap;
    q.unit0 = units;
    units += Mp / 8;  // the quantizer's 8-row units
  }
  qs.total = units;
  // profiling marks; whatever is not handed to the records (an early
  // return, a failed mark) is destroyed on the way out
  struct Marks {
    std::vector<hipEvent_t> v;
    ~Marks() {
      for (hipEvent_t e : v)
        if (e) (void)hipEventDestroy(e);
    }
    bool all(size_t n) const {
      return v.size() == n && std::all_of(v.begin(), v.end(), [](hipEvent_t e) { return e; });
    }
  } marks;
  auto mark = [&]() {
    if (t_prof) marks.v.push_back(prof_mark(s));
  };
  mark();
  hipError_t e = launch_act_quant_segs(qs, s);
  if (e != hipSuccess) return hip_error(e, "stack act_quant launch");
  mark();
  // the independent items (and a folded one): one grouped launch per set
  // with the same K
  std::vector<int> members;
  for (int j = 0; j < ngroup; j++) members.push_back(j);
  if (fold_g >= 0) members.push_back(fold_s);
  std::vector<bool> done(n, false);
  for (size_t a = 0; a < members.size(); a++) {
    const int j = members[a];
    if (done[j] || cv[j].seg < 0) continue;
    GemmGroup g{};
    const sdq_group_item& first = items[j];
    for (size_t b = a; b < members.size(); b++) {
      const int k = members[b];
      const sdq_group_item& it = items[k];
      if (done[k] || cv[k].seg < 0 || !same_group(first, it)) continue;
      done[k] = true;
      const QuantSeg& q = qs.s[cv[k].seg];
      GemmProblem& p = g.p[g.count++];
      p.wt = it.w->frags;
      p.scale = it.w->scale;
      p.bias = q.cc.bias_pad;
      p.gate = q.cc.gate_pad;
      p.at = q.at;
      p.as = q.as;
      p.resid = it.epi.resid;
      p.Y = it.Y;
      p.M = (int)it.M;
      p.N = (int)it.w->N;
      p.kind = it.epi.kind;
      p.gate_fma = it.epi.gate_fma;
      if (fold_g >= 0 && (k == fold_g || k == fold_s)) {  // plain output into scratch
        p.kind = SDQ_EPI_NONE;
        p.gate = nullptr;
        p.resid = nullptr;
        p.Y = base + (k == fold_g ? yg_off : ys_off);
      }
    }
    EpiArgs ea = make_epi(&first.epi, first.w->K);
    ea.bias = ea.gate = ea.resid = nullptr;  // per problem, from the table
    e = launch_qgemm_group(g, first.w->KFp, ea, sink, cu_count, s);
    if (e != hipSuccess) return hip_error(e, "stack grouped qgemm launch");
  }
  if (fold_g >= 0) {
    const sdq_group_item& G = items[fold_g];
    const sdq_group_item& S = items[fold_s];
    const ResidStep ra{reinterpret_cast<const float*>(base + yg_off), G.epi.gate, G.epi.kind,
                       G.epi.gate_fma};
    const ResidStep rb{reinterpret_cast<const float*>(base + ys_off), S.epi.gate, S.epi.kind,
                       S.epi.gate_fma};
    e = launch_resid2(static_cast<float*>(S.Y), S.M, S.w->N, ra, rb, s);
    if (e != hipSuccess) return hip_error(e, "stack residual launch");
  }
  mark();
  // then the others, in order
  int tail = 0;
  for (int i = ngroup; i < n; i++) {
    const sdq_group_item& it = items[i];
    if (cv[i].seg < 0 || (fold_g >= 0 && i == fold_s)) continue;
    const QuantSeg& q = qs.s[cv[i].seg];
    const EpiArgs ea = make_epi(&it.epi, it.w->K);
    const GemmAux aux{q.cc.bias_pad, q.cc.gate_pad, sink, cu_count, 1, nullptr, nullptr, &tail,
                      nullptr};
    e = launch_qgemm(cfgs[i], it.w->frags, it.w->scale, q.at, q.as, it.M, it.w->N, it.w->KFp, ea,
                     it.Y, 1, aux, s);
    if (e != hipSuccess) return hip_error(e, "stack qgemm launch");
  }
  mark();
  if (has_ffn) {
    // fc1 + GELU, writing the hidden state's row maxima, then fc2's quantizer
    // from them and fc2 with the gated residual (as ffn_device)
    const sdq_weight* fc1 = ffn->fc1;
    RowMax rm;
    rm.stride = (int)round_up(std::max(gemm_rmax_chunks(kCfg128x128, fc1->N),
                                       gemm_rmax_chunks(kCfg256x256, fc1->N)),
                              4);
    if ((rc = rmax_buffer(dev, s, (size_t)ffn->M * rm.stride * sizeof(float), &rm.p))) return rc;
    const sdq_epilogue e1{SDQ_EPI_GELU, 1, ffn->b1, nullptr, nullptr};
    EpiArgs ea = make_epi(&e1, fc1->K);
    ea.rmax = rm.p;
    ea.rmax_stride = rm.stride;
    const QuantSeg& q = qs.s[cv[n].seg];
    const GemmAux aux{q.cc.bias_pad, nullptr, sink, cu_count, 1, nullptr, &rm.chunks, &tail,
                      nullptr};
    e = launch_qgemm(cfg1, fc1->frags, fc1->scale, q.at, q.as, ffn->M, fc1->N, fc1->KFp, ea,
                     ffn->hid, 1, aux, s);
    if (e != hipSuccess) return hip_error(e, "stack fc1 launch");
    mark();
    if (marks.all(5)) {
      t_recs.push_back({"act_quant_stack", marks.v[0], marks.v[1]});
      t_recs.push_back({"qgemm_group", marks.v[1], marks.v[2]});
      t_recs.push_back({"qgemm_stack_seq", marks.v[2], marks.v[3]});
      t_recs.push_back({"qgemm_fc1_stack", marks.v[3], marks.v[4]});
      marks.v.clear();
    }
    const sdq_epilogue e2{SDQ_EPI_GATED, ffn->gate_fma, ffn->b2, ffn->gate, ffn->x};
    return qlinear_device(ffn->fc2, ffn->hid, ffn->M, ffn->fc2->K, &e2, ffn->x, s, &rm, nullptr);
  }
  if (marks.all(4)) {
    t_recs.push_back({"act_quant_stack", marks.v[0], marks.v[1]});
    t_recs.push_back({"qgemm_group", marks.v[1], marks.v[2]});
    t_recs.push_back({"qgemm_stack_seq", marks.v[2], marks.v[3]});
    marks.v.clear();
  }
  return SDQ_OK;
}

int sdq_ffn(const sdq_weight* fc1, const float* b1, const sdq_weight* fc2, const float* b2,
            const float* h, int64_t M, const float* gate, int gate_fma, float* hid, float* x,
            void* stream) {
  return ffn_device(fc1, b1, fc2, b2, h, M, gate, gate_fma, hid, x,
                    static_cast<hipStream_t>(stream), nullptr);
}

int sdq_ffn_lnmod(const sdq_weight* fc1, const float* b1, const sdq_weight* fc2, const float* b2,
                  float* x, int64_t M, const float* shift, const float* scale, float eps,
                  const float* gate, int gate_fma, float* hid, void* stream) {
  if (!shift || !scale) return set_error(SDQ_ERR_INVALID, "ffn: null shift or scale");
  const LnMod lm{shift, scale, eps};
  return ffn_device(fc1, b1, fc2, b2, x, M, gate, gate_fma, hid, x,
                    static_cast<hipStream_t>(stream), &lm);
}

int sdq_qlinear_lnmod(const sdq_weight* w, const float* x, int64_t M, int64_t K,
                      const float* shift, const float* scale, float eps,
                      const sdq_epilogue* epi, void* Y, void* stream) {
  if (!shift || !scale) return set_error(SDQ_ERR_INVALID, "null shift or scale");
  const LnMod lm{shift, scale, eps};
  return qlinear_device(w, x, M, K, epi, Y, static_cast<hipStream_t>(stream), nullptr, nullptr,
                        &lm);
}

int sdq_rmsnorm_rope_batch(const sdq_rms_seg* segs, int nseg, int64_t C, int heads, float eps,
                           void* stream) {
  if (nseg < 0 || nseg > SDQ_MAX_RMS_SEGS || (nseg > 0 && !segs))
    return set_error(SDQ_ERR_INVALID, "rmsnorm_rope: 0 to 4 segments");
  if (C <= 0 || heads <= 0 || C % heads != 0 || (C / heads) % 2 != 0)
    return set_error(SDQ_ERR_INVALID, "rmsnorm_rope: need C > 0, C = heads * even head_dim");
  RmsSeg g[SDQ_MAX_RMS_SEGS];
  int n = 0;
  int64_t rows_w = 0;
  for (int i = 0; i < nseg; i++) {
    const sdq_rms_seg& a = segs[i];
    if (a.L < 0) return set_error(SDQ_ERR_INVALID, "negative L");
    if (a.L == 0) continue;
    if (!a.x) return set_error(SDQ_ERR_INVALID, "null x");
    if (!a.w && (a.nr <= 0 || !a.cs))
      return set_error(SDQ_ERR_INVALID, "rmsnorm_rope: nothing to do");
    if (a.ld < C) return set_error(SDQ_ERR_INVALID, "rmsnorm_rope: need ld >= C");
    if (a.nr < 0 || a.nr > C / heads / 2 || (a.nr > 0 && !a.cs))
      return set_error(SDQ_ERR_INVALID, "rmsnorm_rope: need 0 <= nr <= head_dim/2 and a table");
    g[n++] = RmsSeg{a.x, a.L, a.ld, a.w, a.nr > 0 ? a.cs : nullptr, a.nr, nullptr};
    if (a.w) rows_w += a.L;
  }
  if (n == 0) return SDQ_OK;
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  float* inv = nullptr;
  if (rows_w > 0 &&
      (rc = ws_floats(dev, s, &Workspace::rinv, &Workspace::rinv_bytes, (size_t)rows_w * 4, &inv)))
    return rc;
  for (int i = 0; i < n; i++)
    if (g[i].w) {
      g[i].inv = inv;
      inv += g[i].L;
    }
  hipEvent_t p0 = t_prof ? prof_mark(s) : nullptr;
  hipError_t e = launch_rmsnorm_rope_segs(g, n, C, heads, eps, s);
  if (e != hipSuccess) {
    drop_events({p0});
    return hip_error(e, "rmsnorm_rope launch");
  }
  if (t_prof) {
    hipEvent_t p1 = prof_mark(s);
    if (p0 && p1) {
      t_recs.push_back({"rmsnorm_rope", p0, p1});
    } else {
      for (hipEvent_t ev : {p0, p1})
        if (ev) (void)hipEventDestroy(ev);
    }
  }
  return SDQ_OK;
}

int sdq_rmsnorm_rope(float* x, int64_t L, int64_t C, int64_t ld, const float* w, float eps,
                     int heads, const float* cs, int nr, void* stream) {
  const sdq_rms_seg g{x, L, ld, w, cs, nr};
  return sdq_rmsnorm_rope_batch(&g, 1, C, heads, eps, stream);
}

int sdq_layernorm(const float* x, int64_t M, int64_t K, const float* w, const float* b, float eps,
                  float* y, void* stream) {
  if (M < 0 || K < 0) return set_error(SDQ_ERR_INVALID, "negative dims");
  if (M == 0) return SDQ_OK;
  if (K == 0 || !x || !y) return set_error(SDQ_ERR_INVALID, "layernorm: null data or K = 0");
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  float2* st = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    Workspace& ws = g_ws[{dev, s}];
    if ((rc = grow(s, reinterpret_cast<void**>(&ws.st), &ws.st_bytes, (size_t)M * sizeof(float2))))
      return rc;
    st = ws.st;
  }
  hipEvent_t p0 = t_prof ? prof_mark(s) : nullptr;
  hipError_t e = launch_ln_stats(x, M, K, eps, st, s);
  if (e == hipSuccess) e = launch_ln_apply(x, M, K, st, w, b, y, s);
  if (e != hipSuccess) {
    drop_events({p0});
    return hip_error(e, "layernorm launch");
  }
  if (t_prof) {
    hipEvent_t p1 = prof_mark(s);
    if (p0 && p1) {
      t_recs.push_back({"layernorm", p0, p1});
    } else {
      for (hipEvent_t ev : {p0, p1})
        if (ev) (void)hipEventDestroy(ev);
    }
  }
  return SDQ_OK;
}

int sdq_add(float* x, const float* y, int64_t n, void* stream) {
  if (n < 0) return set_error(SDQ_ERR_INVALID, "negative n");
  if (n == 0) return SDQ_OK;
  if (!x || !y) return set_error(SDQ_ERR_INVALID, "add: null pointer");
  hipError_t e = launch_add(x, y, n, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? SDQ_OK : hip_error(e, "add launch");
}

int sdq_linear_f32(const float* x, int64_t M, int64_t K, const float* w, int64_t N,
                   const float* bias, float* y, void* stream) {
  if (M < 0 || K < 0 || N < 0) return set_error(SDQ_ERR_INVALID, "linear_f32: negative dims");
  if (M == 0 || N == 0) return SDQ_OK;
  if (!y || (K > 0 && (!x || !w))) return set_error(SDQ_ERR_INVALID, "linear_f32: null pointer");
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipEvent_t p0 = t_prof ? prof_mark(s) : nullptr;
  const hipError_t e = launch_linear_f32(x, M, K, w, N, bias, y, g_dev[dev].cu_count, s);
  if (e != hipSuccess) {
    drop_events({p0});
    return hip_error(e, "linear_f32 launch");
  }
  if (t_prof) {
    hipEvent_t p1 = prof_mark(s);
    if (p0 && p1) {
      t_recs.push_back({"linear_f32", p0, p1});
    } else {
      for (hipEvent_t ev : {p0, p1})
        if (ev) (void)hipEventDestroy(ev);
    }
  }
  return SDQ_OK;
}

int sdq_sdpa(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v, int64_t ldv,
             float* out, int64_t ldo, int64_t Lq, int64_t Lk, int heads, int head_dim,
             void* stream) {
  return sdq_sdpa_batched(q, ldq, k, ldk, v, ldv, out, ldo, Lq, Lk, heads, head_dim, 1, stream);
}

int sdq_sdpa_batched(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                     int64_t ldv, float* out, int64_t ldo, int64_t Lq, int64_t Lk, int heads,
                     int head_dim, int batch, void* stream) {
  if (Lq < 0 || Lk < 0) return set_error(SDQ_ERR_INVALID, "negative Lq or Lk");
  if (batch < 1 || batch > 65535) return set_error(SDQ_ERR_INVALID, "sdpa: batch must be 1..65535");
  if (Lq == 0) return SDQ_OK;
  if (Lk == 0) return set_error(SDQ_ERR_INVALID, "sdpa: no keys");
  if (head_dim != 128) return set_error(SDQ_ERR_INVALID, "sdpa: head_dim must be 128");
  if (heads <= 0) return set_error(SDQ_ERR_INVALID, "sdpa: heads must be positive");
  if (!q || !k || !v || !out) return set_error(SDQ_ERR_INVALID, "sdpa: null pointer");
  const int64_t C = (int64_t)heads * head_dim;
  if (ldq < C || ldk < C || ldv < C || ldo < C)
    return set_error(SDQ_ERR_INVALID, "sdpa: row strides must cover heads * head_dim");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || ldq % 4 || ldk % 4 ||
      ldv % 4 || ldo % 4)
    return set_error(SDQ_ERR_INVALID, "sdpa: 16-byte aligned rows required");
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int cu_count = g_dev[dev].cu_count;
  float* part = nullptr;
  const int64_t pf = sdpa_part_floats(Lq, Lk, heads, batch, cu_count);
  if (pf > 0 && (rc = ws_floats(dev, s, &Workspace::sdpa_part, &Workspace::sdpa_part_bytes,
                                (size_t)pf * sizeof(float), &part)))
    return rc;
  hipEvent_t p0 = t_prof ? prof_mark(s) : nullptr;
  hipError_t e = launch_sdpa(q, ldq, k, ldk, v, ldv, out, ldo, Lq, Lk, heads, s, batch, part,
                             cu_count);
  if (e != hipSuccess) {
    drop_events({p0});
    return hip_error(e, "sdpa launch");
  }
  if (t_prof) {
    hipEvent_t p1 = prof_mark(s);
    if (p0 && p1) {
      t_recs.push_back({"sdpa", p0, p1});
    } else {
      for (hipEvent_t ev : {p0, p1})
        if (ev) (void)hipEventDestroy(ev);
    }
  }
  return SDQ_OK;
}

int sdq_qgemm(const sdq_weight* w, const float* A, int64_t M, int64_t K, float* Y, void* stream) {
  return qlinear_device(w, A, M, K, nullptr, Y, static_cast<hipStream_t>(stream));
}

int sdq_qlinear_host(const sdq_weight* w, const float* A, int64_t M, int64_t K,
                     const sdq_epilogue* epi, void* Y) {
  int rc = check_weight(w, K);
  if (rc) return rc;
  if ((rc = validate_epi(epi))) return rc;
  if (M < 0) return set_error(SDQ_ERR_INVALID, "negative M");
  const int64_t N = w->N;
  if ((rc = check_rows(M, N, ""))) return rc;
  if (M == 0 || N == 0) return SDQ_OK;
  int dev = -1;
  if ((rc = current_device(&dev))) return rc;
  if ((rc = ensure_device(dev))) return rc;
  HostStage& hs = t_host_stage[dev];
  if ((rc = host_stage_ready(hs))) return rc;
  const size_t abytes = (size_t)(M * K) * 4, ybytes = (size_t)(M * N) * 4;
  // one device block: A | Y | resid | bias | gate, each 256-byte aligned
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  const bool has_resid = epi && epi->resid;
  const size_t o_y = al(abytes), o_r = o_y + al(ybytes), o_b = o_r + (has_resid ? al(ybytes) : 0);
  const size_t o_g = o_b + al((size_t)N * 4), total = o_g + al((size_t)N * 4);
  if (total > hs.dbytes) {
    // the stage's stream is idle here (every call ends synchronized)
    if (hs.dbuf) (void)hipFree(hs.dbuf);
    hs.dbuf = nullptr;
    hs.dbytes = 0;
    hipError_t e = hipMalloc(&hs.dbuf, total);
    if (e != hipSuccess) {
      hs.dbuf = nullptr;
      return hip_error(e, "hipMalloc (host-call buffers)");
    }
    hs.dbytes = total;
  }
  char* buf = hs.dbuf;
  sdq_epilogue de{};
  if (epi) de = *epi;
  rc = host_stage_h2d(hs, buf, A, abytes);
  if (!rc && has_resid) {
    rc = host_stage_h2d(hs, buf + o_r, epi->resid, ybytes);
    de.resid = reinterpret_cast<float*>(buf + o_r);
  }
  if (!rc && epi && epi->bias) {
    rc = host_stage_h2d(hs, buf + o_b, epi->bias, (size_t)N * 4);
    de.bias = reinterpret_cast<float*>(buf + o_b);
  }
  if (!rc && epi && epi->gate) {
    rc = host_stage_h2d(hs, buf + o_g, epi->gate, (size_t)N * 4);
    de.gate = reinterpret_cast<float*>(buf + o_g);
  }
  if (!rc)
    rc = qlinear_device(w, reinterpret_cast<float*>(buf), M, K, epi ? &de : nullptr, buf + o_y,
                        hs.stream);
  if (!rc) rc = host_stage_d2h(hs, Y, buf + o_y, ybytes);
  // leave the stage idle whatever happened
  const hipError_t e = hipStreamSynchronize(hs.stream);
  if (!rc && e != hipSuccess) rc = hip_error(e, "hipStreamSynchronize (host call)");
  return rc;
}

int sdq_act_quant(const float* A, int64_t M, int64_t K, int8_t* aq, float* as, void* stream) {
  if (M < 0 || K < 0) return set_error(SDQ_ERR_INVALID, "negative dims");
  if (M > kMaxRows || K > kMaxWeightK)
    return set_error(SDQ_ERR_INVALID, "act_quant: at most 2^30 rows of at most 2^22 values");
  if (M == 0) return SDQ_OK;
  if (!as || (K > 0 && (!A || !aq))) return set_error(SDQ_ERR_INVALID, "null pointer");
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  if ((rc = ensure_device(dev))) return rc;
  hipError_t e = launch_act_quant_rowmajor(A, M, K, aq, as, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_error(e, "act_quant launch");
  return SDQ_OK;
}

int sdq_device_alloc(size_t bytes, void** out) {
  if (!out) return set_error(SDQ_ERR_INVALID, "null out");
  *out = nullptr;
  hipError_t e = hipMalloc(out, bytes ? bytes : 1);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return set_error(SDQ_ERR_NOMEM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
  }
  return SDQ_OK;
}

int sdq_device_free(void* p) {
  if (!p) return SDQ_OK;
  hipError_t e = hipFree(p);
  if (e != hipSuccess) return hip_error(e, "hipFree");
  return SDQ_OK;
}

int sdq_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  if (bytes == 0) return SDQ_OK;
  if (!dst || !src) return set_error(SDQ_ERR_INVALID, "null pointer");
  hipMemcpyKind k;
  switch (kind) {
    case SDQ_H2D: k = hipMemcpyHostToDevice; break;
    case SDQ_D2H: k = hipMemcpyDeviceToHost; break;
    case SDQ_D2D: k = hipMemcpyDeviceToDevice; break;
    default: return set_error(SDQ_ERR_INVALID, "bad copy kind");
  }
  hipError_t e = hipMemcpyAsync(dst, src, bytes, k, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_error(e, "hipMemcpyAsync");
  return SDQ_OK;
}

int sdq_stream_sync(void* stream) {
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize");
  return SDQ_OK;
}

int sdq_stream_wait(void* waiter, void* signaler) {
  if (waiter == signaler) return SDQ_OK;
  // One event per thread and device, made once and kept: a wait takes the
  // event's latest record at the time of the call, so recording it again
  // later leaves earlier waits alone, and an event a graph capture recorded
  // is never destroyed under it.
  thread_local hipEvent_t t_ev[kMaxDev] = {};
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  hipEvent_t& ev = t_ev[dev];
  hipError_t e = hipSuccess;
  if (!ev) {
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      ev = nullptr;
      return hip_error(e, "hipEventCreateWithFlags");
    }
  }
  e = hipEventRecord(ev, static_cast<hipStream_t>(signaler));
  if (e == hipSuccess) e = hipStreamWaitEvent(static_cast<hipStream_t>(waiter), ev, 0);
  if (e != hipSuccess) return hip_error(e, "stream wait");
  return SDQ_OK;
}

int sdq_profile_begin(void) {
  t_prof = true;
  return SDQ_OK;
}

int sdq_qlinear_noalloc(const sdq_weight* w, const float* A, int64_t M, int64_t K,
                        const sdq_epilogue* epi, void* Y, void* stream) {
  int rc = check_weight(w, K);
  if (rc) return rc;
  if ((rc = ensure_device(w->device))) return rc;
  char* p = nullptr;
  std::string why;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    p = g_dev[w->device].scratch;
    why = g_dev[w->device].scratch_err;
  }
  if (!p) return set_error(SDQ_ERR_HIP, "sdq_qlinear_noalloc: scratch unavailable (" + why + ")");
  return qlinear_device(w, A, M, K, epi, Y, static_cast<hipStream_t>(stream), nullptr, nullptr,
                        nullptr, p);
}

int sdq_qlinear_plan(const sdq_weight* w, int64_t M, int epi_kind, sdq_gemm_plan* out) {
  if (!w || !out) return set_error(SDQ_ERR_INVALID, "null weight or out");
  if (M < 0) return set_error(SDQ_ERR_INVALID, "negative M");
  int rc = check_rows(M, w->N, "");
  if (rc) return rc;
  if ((rc = ensure_device(w->device))) return rc;
  std::memset(out, 0, sizeof(*out));
  out->splitk = 1;
  if (M == 0 || w->N == 0) return SDQ_OK;
  const int cu = g_dev[w->device].cu_count;
  const int cfg = choose_gemm_cfg(M, w->N, w->KFp, epi_kind, cu);
  auto put = [&](const std::string& name, int64_t r0, int64_t rows) {
    const int i = out->nlaunch++;
    std::snprintf(out->name[i], sizeof(out->name[i]), "%s", name.c_str());
    out->row0[i] = r0;
    out->rows[i] = rows;
  };
  if (cfg == kCfgSkinny && qin_fits(M, w->K, w->KFp) && !std::getenv("SDQ_NO_QIN")) {
    put("qgemm_skinny_qin", 0, M);
    return SDQ_OK;
  }
  out->splitk = choose_splitk(cfg, M, w->N, w->KFp, cu);
  const std::string g = std::string("qgemm_") + gemm_cfg_name(cfg) + (out->splitk > 1 ? "_splitk" : "");
  const int64_t Ma = (cfg == kCfg256x256 && w->K > 0) ? tail_split_rows(M, w->N, cu) : 0;
  if (Ma > 0) {
    put(g, 0, Ma);
    put("qgemm_tail128", Ma, M - Ma);
  } else {
    put(g, 0, M);
  }
  return SDQ_OK;
}

int sdq_profile_end(sdq_kernel_time* out, int max_records, int* n_records) {
  t_prof = false;
  std::vector<std::pair<std::string, std::pair<int, double>>> agg;
  std::set<hipEvent_t> owned;
  int rc = SDQ_OK;
  for (const ProfRec& r : t_recs) {
    owned.insert(r.a);
    owned.insert(r.b);
    if (rc != SDQ_OK) continue;
    hipError_t e = hipEventSynchronize(r.b);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.a, r.b);
    if (e != hipSuccess) {
      rc = hip_error(e, "profile events");
      continue;
    }
    auto it = agg.begin();
    for (; it != agg.end(); ++it)
      if (it->first == r.name) break;
    if (it == agg.end()) {
      agg.push_back({r.name, {0, 0.0}});
      it = agg.end() - 1;
    }
    it->second.first += 1;
    it->second.second += ms;
  }
  for (hipEvent_t ev : owned) (void)hipEventDestroy(ev);
  t_recs.clear();
  if (rc != SDQ_OK) return rc;
  int n = 0;
  for (const auto& a : agg) {
    if (out && n < max_records) {
      std::snprintf(out[n].name, sizeof(out[n].name), "%s", a.first.c_str());
      out[n].launches = a.second.first;
      out[n].total_ms = a.second.second;
    }
    n++;
  }
  if (n_records) *n_records = n;
  return SDQ_OK;
}

int sdq_sync(void) {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_error(e, "hipDeviceSynchronize");
  return SDQ_OK;
}

}  // extern "C"
