/*
 * sdq — MI355X (gfx950) int8 qGEMM, C ABI.
 *
 * Drop-in device implementation of the reference's int8 Linear path
 * (JasonHonKL/Self-evolve-diffusion-cpp):
 *
 *   sd::qgemm(const Tensor& A, const Tensor& Bq, const Tensor& bs, Tensor& out)
 *       src/core/tensor.h:48-52, src/core/qgemm.cpp:73-142
 *   mlin(x, Linear, y)  — qgemm + bias pass, src/model/ovi_dit.cpp:66-84
 *   and the consumers that follow mlin in the DiT blocks:
 *       gelu_tanh_inplace  src/model/ovi_dit.cpp:132-142 (after ffn fc1, 217-218)
 *       gated_add_inplace  src/model/ovi_dit.cpp:152-159 (after ffn fc2 / self o, 187, 221)
 *       add_inplace        src/model/ovi_dit.cpp:144-149 (after cross o, 251)
 *   .sdcpp v1 packed weights: src/serde/sdcpp.cpp:1-133 (int8 [N,K] row-major,
 *       then N f32 scales, no alignment padding).
 *
 * Semantics (bit-exact with the reference CPU path):
 *   per row i of A:   mx = max_k |A[i,k]|, sc = mx/127 (1 if 0), inv = 1/sc,
 *                     aq[i,k] = clamp(cvt_rne(A[i,k]*inv), -127, 127)
 *                     (NaN / out-of-int32 products give -127, as x86 cvtss2si)
 *   acc[i,j] = sum_k aq[i,k] * Bq[j,k]             (exact int32)
 *   y[i,j]   = fl( fl((float)acc) * fl(sc_i * bs[j]) )
 *   bias:      y = fl(y + bias[j])
 *   epilogue:  GELU  y = gelu_tanh(y)               (tolerance: the reference uses libm tanh)
 *              GATED x[i,j] = fma(y, gate[j], x[i,j]) (or x + fl(y*gate))
 *              RESID x[i,j] = fl(x[i,j] + y)
 *
 * Conventions: every function returns SDQ_OK (0) or a positive SDQ_ERR_*
 * code and never throws; sdq_last_error() gives the calling thread's last
 * message. Device pointers are plain HIP device addresses; `stream` is a
 * hipStream_t passed as void* (NULL = the null stream). Functions named
 * *_host take host pointers and are synchronous.
 *
 * Size limits (the kernels' in-tile offsets and tile counters are 32-bit):
 * a weight has at most 2^20 outputs (N) and 2^22 inputs (K); a GEMM call has
 * at most 2^30 rows (M) and M*N under 2^40. Larger shapes are refused with
 * SDQ_ERR_INVALID before anything is allocated or launched.
 */
#ifndef SDQ_H_
#define SDQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SDQ_OK 0
#define SDQ_ERR_INVALID 1 /* bad argument or shape */
#define SDQ_ERR_HIP 2     /* HIP runtime error */
#define SDQ_ERR_NOMEM 3   /* device allocation failed */
#define SDQ_ERR_FORMAT 4  /* malformed .sdcpp file */
#define SDQ_ERR_NODEV 5   /* no usable gfx950 device */
#define SDQ_ERR_NOTFOUND 6

/* Epilogue kinds (see semantics above). */
#define SDQ_EPI_NONE 0  /* Y = y (+bias)                                  */
#define SDQ_EPI_GELU 1  /* Y = gelu_tanh(y (+bias))                       */
#define SDQ_EPI_GATED 2 /* Y = fma(y (+bias), gate, resid)                */
#define SDQ_EPI_RESID 3 /* Y = resid + (y (+bias))                        */
#define SDQ_EPI_ACC 4   /* Y (int32*) = raw accumulators, no rescale      */

typedef struct sdq_weight sdq_weight;

typedef struct sdq_epilogue {
  int kind;            /* SDQ_EPI_*                                             */
  int gate_fma;        /* GATED: 1 = fma(y,g,x) (reference -march=native build), */
                       /*        0 = x + fl(y*g)                                 */
  const float* bias;   /* [N] or NULL                                           */
  const float* gate;   /* [N] (GATED)                                           */
  const float* resid;  /* [M,N] residual input (GATED/RESID); may equal Y       */
} sdq_epilogue;

typedef struct sdq_device_info {
  int device;
  int cu_count;
  int max_clock_khz;     /* shader clock as reported by the runtime */
  int mem_clock_khz;
  int64_t total_mem;
  char arch[64];         /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
} sdq_device_info;

/* Thread-local text of the last error raised on this thread ("" if none). */
const char* sdq_last_error(void);

/* Library version string: "sdq <version> gfx950 src:<16 hex digits>", the
 * last field a fingerprint of the device sources and build flags the library
 * was compiled from. */
const char* sdq_version(void);

/* Select `device` for this thread and check it is gfx950. Idempotent.
 * Replaces: nothing (the reference is CPU-only; tensor.cpp:81-83 sizes its
 * thread pool instead). */
int sdq_init(int device);
int sdq_device_info_get(sdq_device_info* out);

/* ---- weights (one-time upload + repack) --------------------------------
 * Upload an int8 [N,K] row-major weight and its N f32 per-row scales from
 * HOST memory (e.g. views into an mmapped .sdcpp file; `scale` may be
 * unaligned, as .sdcpp v1 has no padding) and repack it on the GPU into the
 * MFMA fragment layout. The handle owns the device copy.
 * Replaces: the I8 + ".scale" views of load_sdcpp (src/serde/sdcpp.cpp:107-131)
 * consumed by OviDit::load_impl's lin() (src/model/ovi_dit.cpp:397-415). */
int sdq_weight_upload(const int8_t* q, const float* scale, int64_t N, int64_t K, void* stream,
                      sdq_weight** out);
/* Same from DEVICE memory (q and scale already resident in HBM). */
int sdq_weight_upload_device(const int8_t* q_dev, const float* scale_dev, int64_t N, int64_t K,
                             void* stream, sdq_weight** out);
/* Many weights at once, streamed: each source is 1-4 parts concatenated
 * along N (e.g. q|k|v), host arrays as load_sdcpp yields them (views into the
 * mmapped pack; scales may be unaligned). Host copies into a ring of pinned
 * staging buffers (several threads), asynchronous H2D on a copy stream and the
 * GPU repack of the previous weight overlap. out[i] receives source i's
 * handle; on error no handle is returned. Same device contents as one
 * sdq_weight_upload per (concatenated) weight.
 * Replaces: the per-tensor page-in + lin() + upload of OviDit::load_impl
 * (src/model/ovi_dit.cpp:397-415, 505-530) for a whole pack. */
typedef struct sdq_weight_src {
  int nparts;              /* 1..4 */
  const int8_t* q[4];      /* [rows[i], K] int8, row-major */
  const float* scale[4];   /* [rows[i]] f32, any alignment */
  int64_t rows[4];
  int64_t K;
} sdq_weight_src;
int sdq_weight_upload_batch(const sdq_weight_src* src, int n, void* stream, sdq_weight** out);
/* The same from a .sdcpp file, by file offsets instead of memory views: the
 * parts' int8 rows and scales are read with large sequential reads (several
 * threads) straight into the pinned staging ring, so a cold pack is read
 * from disk once, in order, with no page faults through a mapping.
 * q_off / scale_off: absolute file offsets (the pack index's data and scale
 * offsets; scales right after the int8 rows in .sdcpp v1, any alignment).
 * Same device contents as sdq_weight_upload_batch on the mapped views.
 * Errors: SDQ_ERR_NOTFOUND (cannot open), SDQ_ERR_FORMAT (a part outside the
 * file, a short read).
 * Replaces: the page-in of load_sdcpp's mapped views (src/serde/sdcpp.cpp:
 * 57-60) followed by the per-tensor upload, for a whole pack. */
typedef struct sdq_weight_fsrc {
  int nparts;              /* 1..4 */
  uint64_t q_off[4];       /* [rows[i], K] int8 */
  uint64_t scale_off[4];   /* [rows[i]] f32 */
  int64_t rows[4];
  int64_t K;
} sdq_weight_fsrc;
int sdq_weight_upload_file(const char* path, const sdq_weight_fsrc* src, int n, void* stream,
                           sdq_weight** out);
int sdq_weight_free(sdq_weight* w);
int sdq_weight_dims(const sdq_weight* w, int64_t* N, int64_t* K);
/* Unpack the device copy back to row-major int8 [N,K] + f32 [N] in host
 * memory (repack round-trip check). */
int sdq_weight_export_host(const sdq_weight* w, int8_t* q, float* scale);

/* ---- the qGEMM ---------------------------------------------------------
 * Y[M,N] = epilogue(qgemm(A[M,K], W)), A and Y device pointers (row-major,
 * contiguous). K must equal the weight's K. M == 0 is a no-op; K == 0 gives
 * y = 0 (then bias/epilogue), matching the zero-filled Tensor the reference
 * returns (src/core/qgemm.cpp:74-76). Stream-ordered; no host sync.
 * Scratch (quantized activations, row scales, split-K partials) comes from a
 * workspace per (device, stream) that grows, never shrinks, when a call needs
 * more than any call before it on that stream; growing synchronizes the
 * stream and allocates. Under HIP-graph capture such a call is refused with
 * SDQ_ERR_INVALID before anything is queued (the capture stays usable); one
 * call of the same shape on the stream before the capture makes the captured
 * call allocation-free, and its graph replays bit-identical results.
 * Replaces: sd::qgemm (src/core/tensor.h:52) + mlin's bias pass
 * (src/model/ovi_dit.cpp:66-84) + the consumer named by epi->kind. */
int sdq_qlinear(const sdq_weight* w, const float* A, int64_t M, int64_t K, const sdq_epilogue* epi,
                void* Y, void* stream);

/* Several independent Linears at once: the same results, bit for bit, as one
 * sdq_qlinear per item, with fewer and fuller launches. Items that share K
 * and run on the 128x128 tile path (the medium and small row counts of the
 * DiT's Linears) are quantized by one launch and multiplied by one
 * persistent launch that walks all their tiles, each with its own epilogue;
 * other items run as separate sdq_qlinear calls. For the Linears of a block
 * (or of both branches of a twin layer) that read inputs already computed:
 * q|k|v, cross q, the text k|v, the fusion k|v (ovi_dit.cpp:179-181,
 * 194-196, 235-237, 244-245), or the output projections of two branches.
 * Items must not overlap: no item's Y may be another item's A, resid or Y.
 * n <= SDQ_MAX_GROUP; M == 0 items are skipped. Stream-ordered.
 * Replaces: a sequence of independent mlin calls (ovi_dit.cpp:66-84). */
typedef struct sdq_group_item {
  const sdq_weight* w;
  const float* A;    /* [M, K] device, K = the weight's K */
  int64_t M;
  sdq_epilogue epi;  /* as for sdq_qlinear (resid: this item's own) */
  void* Y;           /* [M, N] device */
} sdq_group_item;
#define SDQ_MAX_GROUP 16
int sdq_qlinear_group(const sdq_group_item* items, int n, void* stream);

/* One DiT block's linear stack when every Linear's input is already there
 * (the attention output, the cross-attention output and the normalized
 * tokens given, as in ovi_dit.cpp:176-222 with the tensors between the
 * Linears as inputs): items[0..ngroup) are independent (as for
 * sdq_qlinear_group), items[ngroup..n) run after them in the given order
 * (e.g. the cross output projection into the x the self-attention output
 * projection just updated), then the FFN when `ffn` is not NULL (as
 * sdq_ffn). Same results as those calls made one after the other, bit for
 * bit; the difference is that every input (the items' A and the FFN's h) is
 * quantized by one launch before any GEMM runs, and that the first later
 * item, when it adds into the output a grouped item adds into (both GATED or
 * RESID in place, same shape), joins the grouped launch: the two plain
 * outputs go to scratch and one elementwise pass applies both residual steps
 * in order. So no output (an item's Y,
 * the FFN's hid or x) may overlap any of those inputs, and no output of the
 * first ngroup items may overlap another of their outputs or residuals
 * (SDQ_ERR_INVALID). Replaces: the separate mlin calls of block_self_fwd,
 * fusion_cross_ffn and ffn_fwd (ovi_dit.cpp:176-222). */
typedef struct sdq_ffn_item {
  const sdq_weight* fc1; /* [F, D] */
  const float* b1;       /* [F] or NULL */
  const sdq_weight* fc2; /* [D, F] */
  const float* b2;       /* [D] or NULL */
  const float* h;        /* [M, D] */
  int64_t M;
  const float* gate;     /* [D] */
  int gate_fma;
  float* hid;            /* [M, F] (written) */
  float* x;              /* [M, D] updated in place */
} sdq_ffn_item;
int sdq_qlinear_stack(const sdq_group_item* items, int n, int ngroup, const sdq_ffn_item* ffn,
                      void* stream);

/* sdq_qlinear for callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * It can be captured into a HIP graph with no warm-up call. The same results as sdq_qlinear, bit for
 * bit, with no hipMalloc / hipFree or other allocation on any call: the
 * quantized activations and the GEMM's other scratch live in a static device
 * array of SDQ_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends).
 * Limit: the call's scratch (about M*K bytes of quantized activations, plus
 * 8*N bytes and, for split-K shapes, up to 32*M*N bytes) must fit that array, e.g.
 * up to 4096 rows at K = 14336 or 20480 rows at K = 3072; larger calls fail
 * with SDQ_ERR_INVALID before anything is launched. Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (different streams,
 * threads) race; serialize them. No profiling records are made. */
#define SDQ_NOALLOC_SCRATCH_BYTES (64u << 20)
int sdq_qlinear_noalloc(const sdq_weight* w, const float* A, int64_t M, int64_t K,
                        const sdq_epilogue* epi, void* Y, void* stream);

/* The FFN of a DiT block after its norm (src/model/ovi_dit.cpp:218-221,
 * ffn_fwd):  hid = gelu_tanh(mlin(h, fc1));  x = fma(mlin(hid, fc2), gate, x)
 * (gate_fma = 0: x + fl(y*gate)). fc1 is [F,D], fc2 [D,F]; h and x are
 * [M,D], hid [M,F] (written), all device pointers; x is updated in place.
 * Same results as sdq_qlinear(fc1, GELU) then sdq_qlinear(fc2, GATED), bit
 * for bit; faster: fc1's epilogue passes hid's row maxima to fc2's
 * activation quantizer, which then reads hid once.
 * Replaces: mlin + gelu_tanh_inplace + mlin + gated_add_inplace (218-221). */
int sdq_ffn(const sdq_weight* fc1, const float* b1, const sdq_weight* fc2, const float* b2,
            const float* h, int64_t M, const float* gate, int gate_fma, float* hid, float* x,
            void* stream);

/* The DiT's norm + modulation folded into the activation quantizer:
 *   Y = epilogue(qgemm(mod_rows(layernorm(x, eps), shift, scale), W))
 * for the Linears that read a normalized, modulated copy of the residual
 * stream: q|k|v after norm1 (src/model/ovi_dit.cpp:208-210) and ffn fc1
 * after norm2 (216-218). layernorm is blk::layernorm without affine
 * (src/model/blocks.cpp:18-43), mod_rows is x*(1+scale)+shift
 * (ovi_dit.cpp:161-172); both bit-exact with the reference build (serial
 * float sums in k order; mod_rows as one fused multiply-add). shift, scale:
 * [K] device vectors; the normalized rows are never written to memory. */
int sdq_qlinear_lnmod(const sdq_weight* w, const float* x, int64_t M, int64_t K,
                      const float* shift, const float* scale, float eps,
                      const sdq_epilogue* epi, void* Y, void* stream);

/* ffn_fwd whole (src/model/ovi_dit.cpp:214-222): h = mod_rows(layernorm(x),
 * shift, scale); hid = gelu_tanh(mlin(h, fc1)); x = fma(mlin(hid, fc2),
 * gate, x). x [M,D] is the norm's input and the residual, updated in place;
 * hid [M,F] is written. Same bits as sdq_ffn on the reference's h. */
int sdq_ffn_lnmod(const sdq_weight* fc1, const float* b1, const sdq_weight* fc2, const float* b2,
                  float* x, int64_t M, const float* shift, const float* scale, float eps,
                  const float* gate, int gate_fma, float* hid, void* stream);

/* The q / k glue between the q|k|v GEMM and the attention
 * (src/model/ovi_dit.cpp:182-185): in place on L rows of x (row stride ld
 * floats, C columns, e.g. the q or k columns of a q|k|v row),
 *   x = rmsnorm(x, w, eps)        src/core/tensor.cpp:112-123
 *   x = apply_rope(x, heads)      src/model/blocks.cpp:86-100
 * where cs [L][nr][2] holds (cosf, sinf) of each token's nr rotated pair
 * angles (the reference's RopeFreqs.ang through the same libm calls, done by
 * the caller); nr = 0 / cs = NULL skips the rotation (cross-attention q, k),
 * w = NULL skips the rmsnorm (the fusion attention's late rotation of q,
 * ovi_dit.cpp:247). Bit-exact with the reference build. Stream-ordered. */
int sdq_rmsnorm_rope(float* x, int64_t L, int64_t C, int64_t ld, const float* w, float eps,
                     int heads, const float* cs, int nr, void* stream);

/* Several column blocks in one call, e.g. the q and k blocks of q|k|v with
 * their own weights, or cross q, context k and fusion k: the same as
 * sdq_rmsnorm_rope on each, but their serial row sums run side by side in one
 * launch. Segments with L = 0 are skipped. */
typedef struct sdq_rms_seg {
  float* x;        /* first column of the block, rows of stride ld */
  int64_t L;       /* rows */
  int64_t ld;      /* row stride (floats), >= C */
  const float* w;  /* [C] rmsnorm weight, or NULL: rotation only */
  const float* cs; /* [L, nr, 2] (cos, sin) table, or NULL: no rotation */
  int nr;          /* pairs rotated per head */
} sdq_rms_seg;
#define SDQ_MAX_RMS_SEGS 4
int sdq_rmsnorm_rope_batch(const sdq_rms_seg* segs, int nseg, int64_t C, int heads, float eps,
                           void* stream);

/* blk::layernorm (src/model/blocks.cpp:18-43) on the GPU, bit-exact with the
 * reference build: y = fmaf(fl((x - mu)*inv), w, b) with serial-sum row
 * statistics; w, b nullable (1, 0). x, y [M,K] contiguous device arrays
 * (may be the same). Used for the fusion target's pre-norm (ovi_dit.cpp:243)
 * and norm3 (263). */
int sdq_layernorm(const float* x, int64_t M, int64_t K, const float* w, const float* b, float eps,
                  float* y, void* stream);

/* x += y elementwise (add_inplace, src/model/ovi_dit.cpp:144-149), n floats. */
int sdq_add(float* x, const float* y, int64_t n, void* stream);

/* Scaled dot-product attention, non-causal (src/model/blocks.cpp:112-199
 * sdpa, called by ovi_dit.cpp:186, 200, 241, 249): for every head h,
 *   out[i, h] = sum_j softmax_j(q[i, h] . k[j, h] / sqrt(head_dim)) v[j, h]
 * with q [Lq, ldq], k, v [Lk, ldk / ldv], out [Lq, ldo] row-major (e.g. the
 * q, k, v column blocks of a q|k|v tensor), head h in columns
 * h*head_dim .. h*head_dim+head_dim-1; head_dim = 128. Scores as three
 * split fp16 MFMA products per fp32 product (each q and k row scaled by a
 * power of two first, taken back out exactly), P.V as three split bf16 MFMA
 * products, an online softmax: within 2e-5 of the reference's output scale
 * (its serial sums are not reproduced). 16-byte aligned rows. Stream-ordered. */
int sdq_sdpa(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v, int64_t ldv,
             float* out, int64_t ldo, int64_t Lq, int64_t Lk, int heads, int head_dim,
             void* stream);

/* sdq_sdpa over `batch` sequences stacked along the rows: sequence b's
 * queries are rows [b*Lq, (b+1)*Lq) of q (and of out), its keys and values
 * rows [b*Lk, (b+1)*Lk) of k and v; each sequence attends only to its own
 * keys, as `batch` separate sdq_sdpa calls would (same results, bit for
 * bit), in one launch. For the conditional and unconditional forwards of a
 * classifier-free-guidance step run as one stacked forward (the two passes
 * of denoise.cpp:95-98, each with its own text context).
 * Replaces: the sdpa calls of two OviDit::forward passes (ovi_dit.cpp:186,
 * 200, 241, 249). */
int sdq_sdpa_batched(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                     int64_t ldv, float* out, int64_t ldo, int64_t Lq, int64_t Lk, int heads,
                     int head_dim, int batch, void* stream);

/* The F32 branch of mlin (src/model/ovi_dit.cpp:80-82 -> blk::linear,
 * src/model/blocks.cpp:14-16 -> sd::matmul, src/core/gemm.cpp:115-160), for
 * the Linears a pack keeps in fp32 (the audio head [20, 3072]):
 *   y[M,N] = x[M,K] . w[K,N] (+ bias[N])
 * with w in the [in, out] layout lin() gives F32 weights (transp2d,
 * ovi_dit.cpp:409). Bit-exact with the reference's matmul: per output one
 * fused multiply-add chain over k in order from +0 (gemm.cpp:45-75), then
 * fl(c + bias) (add_bias, gemm.cpp:33-40); K == 0 gives 0 (+ bias). The
 * OpenBLAS route the reference takes above 64M multiply-adds in an OpenBLAS
 * build sums in another order and is not reproduced. bias nullable; x, w,
 * bias, y device arrays (y must not overlap x or w). Stream-ordered.
 * Replaces: blk::linear / sd::matmul for F32 Linears. */
int sdq_linear_f32(const float* x, int64_t M, int64_t K, const float* w, int64_t N,
                   const float* bias, float* y, void* stream);

/* Plain sd::qgemm: Y = qgemm(A, W) with no bias (src/core/qgemm.cpp:73). */
int sdq_qgemm(const sdq_weight* w, const float* A, int64_t M, int64_t K, float* Y, void* stream);

/* Host-pointer synchronous variant of sdq_qlinear: copies A (and bias /
 * gate / resid) in, runs, copies Y out. Replaces sd::qgemm's host-tensor
 * contract (tensor.h:52) for callers that hold CPU tensors. Each calling
 * thread keeps, per device, a stream of its own, two 16 MiB pinned bounce
 * buffers and a device buffer that grows to the largest call's inputs and
 * output; they are reused by its later calls (no allocation once grown) and
 * are not released when the thread exits, so call it from long-lived
 * threads. */
int sdq_qlinear_host(const sdq_weight* w, const float* A, int64_t M, int64_t K,
                     const sdq_epilogue* epi, void* Y);

/* ---- activation quantizer (exposed for parity checks and for callers
 * that quantize once and reuse) ------------------------------------------
 * Row-major output: aq [M,K] int8, as [M] f32 (src/core/qgemm.cpp:82-96). */
int sdq_act_quant(const float* A, int64_t M, int64_t K, int8_t* aq, float* as, void* stream);

/* ---- device memory, for host code that reaches HIP only through this ABI */
#define SDQ_H2D 0
#define SDQ_D2H 1
#define SDQ_D2D 2
int sdq_device_alloc(size_t bytes, void** out);
int sdq_device_free(void* p);
/* Stream-ordered copy; `kind` is SDQ_H2D / SDQ_D2H / SDQ_D2D. */
int sdq_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream);
int sdq_stream_sync(void* stream);
/* Work enqueued on `waiter` after this call starts only after the work
 * enqueued on `signaler` before it has finished (an event recorded on
 * signaler, waited on by waiter; the host does not block). The same stream
 * twice: nothing to do. The event is one per host thread and device, kept
 * for the life of the process, so the call can be captured into a graph (it
 * then joins the two streams in the capture). No counterpart in the reference (one CPU thread pool,
 * no streams): the twin-layer pair forward forks the two branches' FFNs onto
 * two streams and joins them with it. */
int sdq_stream_wait(void* waiter, void* signaler);

/* ---- per-kernel timing -------------------------------------------------
 * Between sdq_profile_begin() and sdq_profile_end(), every kernel this
 * thread launches through sdq is bracketed by HIP events recorded on its
 * launch stream. sdq_profile_end() waits for them and returns one record per
 * kernel name (launch count, summed device milliseconds). */
typedef struct sdq_kernel_time {
  char name[48];
  int launches;
  double total_ms;
} sdq_kernel_time;
int sdq_profile_begin(void);
int sdq_profile_end(sdq_kernel_time* out, int max_records, int* n_records);

/* The GEMM launches sdq_qlinear makes for M rows against w (16-byte aligned
 * operands, N % 4 == 0): one, or two when a 256x256 launch hands its last
 * rows to a 128x128 launch; for each, the record name sdq_profile_end uses
 * and the activation rows [row0, row0 + rows) it covers, so a caller can
 * price each kernel's own work. No GPU work is done.
 * Replaces: nothing in the reference (measurement support). */
typedef struct sdq_gemm_plan {
  int nlaunch;
  int splitk;        /* split-K factor (1 = none) */
  char name[2][48];
  int64_t row0[2];
  int64_t rows[2];
} sdq_gemm_plan;
int sdq_qlinear_plan(const sdq_weight* w, int64_t M, int epi_kind, sdq_gemm_plan* out);

/* Synchronize the current device (convenience for ctypes callers). */
int sdq_sync(void);

#ifdef __cplusplus
}
#endif

#endif /* SDQ_H_ */
