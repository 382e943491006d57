/*
 * CPU ORACLE — test infrastructure only.
 *
 * A plain-C restatement of the reference's int8 qGEMM path, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the CHECKER.
 * Nothing in the shipped library links, loads or calls this file: the GPU
 * product path fails loudly when its HIP library is missing instead of
 * falling back here.
 *
 * Every function cites the reference file:line it follows
 * (reference = JasonHonKL/Self-evolve-diffusion-cpp).
 *
 * Parity pins (what checks each function, see tests/test_oracle.py):
 *   orc_act_quant        - compiled reference sd::qgemm (oracle/_ref) bit-exact,
 *                          closed-form special cases (zero row, +-amax -> +-127,
 *                          NaN/Inf/denormal rows), brute-force numpy restatement.
 *   orc_qgemm_acc        - brute-force int64 numpy matmul (exact integer sum).
 *   orc_linear_at        - equal to orc_qgemm + orc_bias_add / orc_gated_add /
 *                          orc_add at every position of small products (so
 *                          pinned through them).
 *   orc_qgemm            - compiled reference sd::qgemm (oracle/_ref) bit-exact on
 *                          many shapes incl. M>=2048 (widen path) and M<2048;
 *                          reference golden vectors (cosine > 0.999 vs fp32).
 *   orc_bias_add         - closed form fl(y+b) vs numpy float32 add.
 *   orc_gated_add        - closed form fma(y,g,x): checked against float64
 *                          y*g+x rounded once (exact for fp32 inputs).
 *   orc_add              - numpy float32 add.
 *   orc_gelu_tanh        - float64 closed form within tolerance only.
 *   orc_layernorm(_affine) - compiled reference blk::layernorm (oracle/_ref)
 *                          bit-exact, with and without the affine, incl. zero,
 *                          constant, tiny and huge rows;
 *                          float64 closed form within tolerance.
 *   orc_mod_rows         - compiled reference mod_rows (oracle/_ref) bit-exact;
 *                          float64 x*(1+h)+s rounded once.
 *   orc_rmsnorm          - compiled reference sd::rmsnorm (oracle/_ref) bit-exact;
 *                          float64 closed form within tolerance.
 *   orc_rope, orc_rope_cs - compiled reference blk::apply_rope bit-exact; rotation
 *                          preserves each pair's norm (float64 check); angle 0 is
 *                          the identity.
 *   orc_sdpa             - compiled reference blk::sdpa (oracle/_ref) bit-exact
 *                          (AVX2 path); float64 softmax attention within
 *                          tolerance; rows of p sum to 1.
 *   orc_rope_freqs_3d/1d - compiled reference rope_freqs_3d / rope_freqs_1d
 *                          bit-exact; float64 closed form within tolerance.
 *   (layernorm, mod_rows, rmsnorm, rope, rope_freqs, sdpa are also pinned to
 *   committed outputs of the reference build, tests/golden/ref_glue.npz, so
 *   the pins hold where the reference sources are absent.)
 *   orc_quantize_rowwise - compiled reference sd::quantize_rowwise bit-exact,
 *                          reference golden replica (lround) bit-exact.
 *   orc_quant_rows       - closed form of the packer's numpy expression
 *                          (float32 semantics) evaluated by numpy itself.
 *   orc_linear_f32       - compiled reference sd::matmul (oracle/_ref, AVX2+FMA
 *                          path) bit-exact, incl. K = 0, no bias, -0 bias,
 *                          denormal products; exact rational evaluation of
 *                          the fma chain (each step rounded once) on tiny
 *                          cases; exact integer dot products when every
 *                          partial sum is an integer below 2^24; committed
 *                          outputs of the reference build
 *                          (tests/golden/ref_linear_f32.npz).
 *   orc_randu            - compiled reference sd::randu bit-exact.
 *   orc_randn            - closed-form splitmix64 + Box-Muller in numpy float64.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; no -ffast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>

/* x86 cvtss2si under the default MXCSR (round-to-nearest-even): NaN and any
 * value whose rounded result does not fit int32 give INT32_MIN (the "integer
 * indefinite" value). The reference's round_to_i8 (src/core/qgemm.cpp:62-69)
 * uses _mm_cvtss_si32 on AVX2 builds (Makefile:4 builds with -march=native). */
static int32_t cvt_rne_i32(float y) {
  if (isnan(y)) return INT32_MIN;
  float r = rintf(y); /* FE_TONEAREST: ties to even */
  if (!(r >= -2147483648.0f && r < 2147483648.0f)) return INT32_MIN;
  return (int32_t)r;
}

/* src/core/qgemm.cpp:62-69 round_to_i8: clamp(cvtss2si(x), -127, 127). */
int orc_round_to_i8(float x) {
  int32_t v = cvt_rne_i32(x);
  if (v < -127) v = -127;
  if (v > 127) v = 127;
  return (int)v;
}

/* src/core/qgemm.cpp:84-96: per-row dynamic activation quantization.
 *   mx  = max_k |r_k|        (std::max(mx, fabs(r)) keeps mx when r is NaN)
 *   sc  = mx / 127.f ; sc == 0 -> 1
 *   inv = 1.f / sc
 *   q_k = round_to_i8(r_k * inv)
 * aq is row-major [M,K], as is [M]. */
void orc_act_quant(const float* A, int64_t M, int64_t K, int8_t* aq, float* as) {
  for (int64_t i = 0; i < M; i++) {
    const float* r = A + i * K;
    float mx = 0.f;
    for (int64_t k = 0; k < K; k++) {
      float a = fabsf(r[k]);
      mx = (mx < a) ? a : mx; /* std::max(mx, a) */
    }
    float sc = mx / 127.f;
    if (sc == 0.f) sc = 1.f;
    as[i] = sc;
    const float inv = 1.f / sc;
    for (int64_t k = 0; k < K; k++) aq[i * K + k] = (int8_t)orc_round_to_i8(r[k] * inv);
  }
}

/* src/core/qgemm.cpp:22-59, 107-138: acc[i,j] = sum_k aq[i,k]*bq[j,k] in
 * int32 (exact for K <= 133k; the widened s16 and the narrow s8 paths give the
 * same integer). */
typedef struct {
  const int8_t* aq; const int8_t* bq; int32_t* acc;
  int64_t M, N, K, j0, j1;
} acc_job;

static void* acc_worker(void* p) {
  acc_job* jb = (acc_job*)p;
  const int64_t K = jb->K, N = jb->N;
  for (int64_t i = 0; i < jb->M; i++) {
    const int8_t* a = jb->aq + i * K;
    for (int64_t j = jb->j0; j < jb->j1; j++) {
      const int8_t* b = jb->bq + j * K;
      int32_t s = 0;
      for (int64_t k = 0; k < K; k++) s += (int32_t)a[k] * (int32_t)b[k];
      jb->acc[i * N + j] = s;
    }
  }
  return NULL;
}

void orc_qgemm_acc(const int8_t* aq, const int8_t* bq, int64_t M, int64_t N, int64_t K,
                   int32_t* acc, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 64) nthreads = 64;
  pthread_t th[64];
  acc_job jobs[64];
  int64_t per = (N + nthreads - 1) / nthreads;
  int n = 0;
  for (int t = 0; t < nthreads; t++) {
    int64_t j0 = t * per, j1 = j0 + per;
    if (j1 > N) j1 = N;
    if (j0 >= j1) break;
    jobs[n] = (acc_job){aq, bq, acc, M, N, K, j0, j1};
    n++;
  }
  for (int t = 1; t < n; t++) pthread_create(&th[t], NULL, acc_worker, &jobs[t]);
  if (n > 0) acc_worker(&jobs[0]);
  for (int t = 1; t < n; t++) pthread_join(th[t], NULL);
}

/* src/core/qgemm.cpp:123-124, 135: out = (float)acc * (as[i] * bs[j]).
 * Two roundings in this order, no fused multiply-add. */
void orc_rescale(const int32_t* acc, const float* as, const float* bs, int64_t M, int64_t N,
                 float* out) {
  for (int64_t i = 0; i < M; i++)
    for (int64_t j = 0; j < N; j++) {
      float s = as[i] * bs[j];
      float a = (float)acc[i * N + j];
      out[i * N + j] = a * s;
    }
}

/* orc_qgemm_acc + orc_rescale, then the mlin bias (src/model/ovi_dit.cpp:71-79,
 * when b is non-null) and the consumer's epilogue, evaluated only at the
 * `count` output positions (ms[i], ns[i]), for spot checks of full-size
 * products. epi: 0 none, 2 gated residual x + y*g (fused multiply-add when
 * gate_fma, as orc_gated_add), 3 plain residual x + y (orc_add); x is the
 * residual row-major [*, N] at resid[m*N + n]. */
void orc_linear_at(const int8_t* aq, const float* as, const int8_t* bq, const float* bs,
                   const float* b, int epi, int gate_fma, const float* gate, const float* resid,
                   int64_t K, int64_t N, const int64_t* ms, const int64_t* ns, int64_t count,
                   float* out) {
  for (int64_t i = 0; i < count; i++) {
    const int64_t m = ms[i], n = ns[i];
    const int8_t* ar = aq + m * K;
    const int8_t* br = bq + n * K;
    int32_t acc = 0;
    for (int64_t k = 0; k < K; k++) acc += (int32_t)ar[k] * (int32_t)br[k];
    float s = as[m] * bs[n];
    float a = (float)acc;
    float y = a * s;
    if (b) y = y + b[n];
    if (epi == 2) {
      const float x = resid[m * N + n];
      if (gate_fma) {
        y = fmaf(y, gate[n], x);
      } else {
        float p = y * gate[n];
        y = x + p;
      }
    } else if (epi == 3) {
      y = resid[m * N + n] + y;
    }
    out[i] = y;
  }
}

/* src/core/qgemm.cpp:73-142 sd::qgemm: out [M,N] (zero-filled first by the
 * Tensor constructor, src/core/tensor.cpp:19-24; M,N or K == 0 returns the
 * zeros, qgemm.cpp:75-76). */
int orc_qgemm(const float* A, const int8_t* Bq, const float* bs, int64_t M, int64_t K, int64_t N,
              float* out, int nthreads) {
  memset(out, 0, (size_t)(M * N) * sizeof(float));
  if (M == 0 || N == 0 || K == 0) return 0;
  int8_t* aq = (int8_t*)malloc((size_t)(M * K) + 1);
  float* as = (float*)malloc((size_t)M * sizeof(float) + 4);
  int32_t* acc = (int32_t*)malloc((size_t)(M * N) * sizeof(int32_t) + 4);
  if (!aq || !as || !acc) { free(aq); free(as); free(acc); return -1; }
  orc_act_quant(A, M, K, aq, as);
  orc_qgemm_acc(aq, Bq, M, N, K, acc, nthreads);
  orc_rescale(acc, as, bs, M, N, out);
  free(aq); free(as); free(acc);
  return 0;
}

/* src/model/ovi_dit.cpp:71-79 (mlin bias pass): y[i,j] += b[j]. */
void orc_bias_add(float* y, const float* b, int64_t M, int64_t N) {
  for (int64_t i = 0; i < M; i++)
    for (int64_t j = 0; j < N; j++) y[i * N + j] = y[i * N + j] + b[j];
}

/* src/model/ovi_dit.cpp:152-159 gated_add_inplace: x += y * gate[c].
 * The reference Makefile builds with -O3 -march=native and GCC's C++ default
 * -ffp-contract=fast, which contracts this to one fused multiply-add
 * (use_fma=1). use_fma=0 restates a build without FMA: x + fl(y*g). */
void orc_gated_add(float* x, const float* y, const float* g, int64_t M, int64_t N, int use_fma) {
  for (int64_t i = 0; i < M; i++)
    for (int64_t j = 0; j < N; j++) {
      int64_t o = i * N + j;
      if (use_fma) x[o] = fmaf(y[o], g[j], x[o]);
      else { float p = y[o] * g[j]; x[o] = x[o] + p; }
    }
}

/* The F32 branch of mlin (src/model/ovi_dit.cpp:80-82): blk::linear
 * (src/model/blocks.cpp:14-16) -> sd::matmul (src/core/gemm.cpp:115-160) as
 * the reference build runs it without OpenBLAS (or below its 64M
 * multiply-add threshold, gemm.cpp:16, 132): row_group (gemm.cpp:45-75)
 * clears each output's accumulator to +0 and adds one fused multiply-add per
 * k in order; add_bias (gemm.cpp:33-40) then adds b[j] in a separate pass.
 * K == 0 leaves the zero output (+ bias, gemm.cpp:123-126).
 * x [M,K], w [K,N] (lin()'s transposed layout, ovi_dit.cpp:409), bias
 * nullable, y [M,N]. */
void orc_linear_f32(const float* x, int64_t M, int64_t K, const float* w, int64_t N,
                    const float* bias, float* y) {
  for (int64_t i = 0; i < M; i++)
    for (int64_t j = 0; j < N; j++) {
      float c = 0.f;
      for (int64_t k = 0; k < K; k++) c = fmaf(x[i * K + k], w[k * N + j], c);
      if (bias) c = c + bias[j];
      y[i * N + j] = c;
    }
}

/* src/model/ovi_dit.cpp:144-149 add_inplace: x += y. */
void orc_add(float* x, const float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) x[i] = x[i] + y[i];
}

/* src/model/blocks.cpp:18-43 blk::layernorm with w = b = nullptr (the DiT's
 * norm1 / norm2 before the self-attention and the FFN, ovi_dit.cpp:208, 216),
 * as the reference build compiles it (pinned against oracle/_ref): the mean
 * and the variance are serial float sums in k order; the variance adds the
 * rounded d*d (not contracted); inv = 1/sqrtf(var/N + eps); the output is
 * (x - mu)*inv*1 + 0 (the +0 turns -0 into +0). */
void orc_layernorm_affine(const float* x, int64_t M, int64_t N, const float* w, const float* b,
                          float eps, float* y);
void orc_layernorm(const float* x, int64_t M, int64_t N, float eps, float* y) {
  orc_layernorm_affine(x, M, N, NULL, NULL, eps, y);
}

/* The same with the affine (w, b nullable: 1 and 0), as the reference build
 * contracts its output: y = fmaf(fl((x - mu)*inv), w, b) (pinned against
 * oracle/_ref; with w = 1, b = 0 this is t + 0). */
void orc_layernorm_affine(const float* x, int64_t M, int64_t N, const float* w, const float* b,
                          float eps, float* y) {
  for (int64_t i = 0; i < M; i++) {
    const float* r = x + i * N;
    float mu = 0.f;
    for (int64_t k = 0; k < N; k++) mu = mu + r[k];
    mu = mu / (float)N;
    float var = 0.f;
    for (int64_t k = 0; k < N; k++) {
      const float d = r[k] - mu;
      const float dd = d * d;
      var = var + dd;
    }
    const float inv = 1.f / sqrtf(var / (float)N + eps);
    for (int64_t k = 0; k < N; k++) {
      const float t = (r[k] - mu) * inv;
      y[i * N + k] = fmaf(t, w ? w[k] : 1.f, b ? b[k] : 0.f);
    }
  }
}

/* src/model/ovi_dit.cpp:161-172 mod_rows: y = x*(1+scale)+shift with scale,
 * shift [C] broadcast over rows; the reference build contracts it to
 * fmaf(x, 1+scale, shift) (pinned against oracle/_ref). */
void orc_mod_rows(const float* x, const float* shift, const float* scale, int64_t L, int64_t C,
                  float* y) {
  for (int64_t l = 0; l < L; l++)
    for (int64_t c = 0; c < C; c++) {
      const float a = 1.f + scale[c];
      y[l * C + c] = fmaf(x[l * C + c], a, shift[c]);
    }
}

/* src/core/tensor.cpp:112-123 rmsnorm, in place over the last dim, as the
 * reference build compiles it (pinned against oracle/_ref): ss is a serial
 * float sum of the rounded r*r (not contracted); inv = 1/sqrtf(ss/N + eps);
 * r = fl(fl(r*inv)*w). Rows of stride ld (>= N). */
void orc_rmsnorm(float* x, int64_t M, int64_t N, int64_t ld, const float* w, float eps) {
  for (int64_t i = 0; i < M; i++) {
    float* r = x + i * ld;
    float ss = 0.f;
    for (int64_t k = 0; k < N; k++) {
      const float rr = r[k] * r[k];
      ss = ss + rr;
    }
    const float inv = 1.f / sqrtf(ss / (float)N + eps);
    for (int64_t k = 0; k < N; k++) {
      const float t = r[k] * inv;
      r[k] = t * w[k];
    }
  }
}

/* (cos, sin) of n rotation angles, as apply_rope evaluates them
 * (src/model/blocks.cpp:93: std::cos / std::sin of a float = cosf / sinf). */
void orc_rope_cs(const float* ang, int64_t n, float* cs) {
  for (int64_t i = 0; i < n; i++) {
    cs[2 * i] = cosf(ang[i]);
    cs[2 * i + 1] = sinf(ang[i]);
  }
}

/* src/model/blocks.cpp:86-100 apply_rope with the (cos, sin) table of
 * orc_rope_cs: pair j < nr of each head turns by its angle; the reference
 * build contracts the rotation to q0 = fmaf(r0, c, -fl(r1*s)),
 * q1 = fmaf(r0, s, fl(r1*c)) (pinned against oracle/_ref). Rows of stride
 * ld, C = heads * head_dim columns. */
void orc_rope(float* x, int64_t L, int64_t C, int64_t ld, int heads, const float* cs, int nr) {
  const int64_t hd = C / heads;
  for (int64_t l = 0; l < L; l++)
    for (int h = 0; h < heads; h++)
      for (int j = 0; j < nr; j++) {
        const float c = cs[2 * (l * nr + j)], s = cs[2 * (l * nr + j) + 1];
        float* q = x + l * ld + h * hd + 2 * j;
        const float r0 = q[0], r1 = q[1];
        const float r1s = r1 * s, r1c = r1 * c;
        q[0] = fmaf(r0, c, -r1s);
        q[1] = fmaf(r0, s, r1c);
      }
}

/* src/model/blocks.cpp:46-67 rope_freqs_3d: angles [T*H*W][n_rot] of the
 * t, h, w axes (t_real = d - 4*(d/6), s_real = 2*(d/6); freq_j =
 * powf(theta, -2j/real)); returns n_rot. */
int orc_rope_freqs_3d(int T, int H, int W, int d, float theta, float* ang) {
  const int t_real = d - 4 * (d / 6), s_real = 2 * (d / 6);
  const int ct = t_real / 2, cs = s_real / 2, nr = ct + 2 * cs;
  float ft[4096], fs[4096];
  if (ct > 4096 || cs > 4096) return -1;
  for (int j = 0; j < ct; j++) ft[j] = powf(theta, (-2.f * (float)j) / (float)t_real);
  for (int j = 0; j < cs; j++) fs[j] = powf(theta, (-2.f * (float)j) / (float)s_real);
  for (int t = 0; t < T; t++)
    for (int h = 0; h < H; h++)
      for (int w = 0; w < W; w++) {
        float* r = ang + (((int64_t)t * H + h) * W + w) * nr;
        int j = 0;
        for (; j < ct; j++) r[j] = (float)t * ft[j];
        for (; j < ct + cs; j++) r[j] = (float)h * fs[j - ct];
        for (; j < nr; j++) r[j] = (float)w * fs[j - ct - cs];
      }
  return nr;
}

/* src/model/blocks.cpp:69-84 rope_freqs_1d (audio): the t-axis part only,
 * angle = fl(fl(l * scaling) * powf(theta, -2j/t_real)); returns n_rot. */
int orc_rope_freqs_1d(int L, int d, float theta, float scaling, float* ang) {
  const int t_real = d - 4 * (d / 6), nr = t_real / 2;
  for (int l = 0; l < L; l++)
    for (int j = 0; j < nr; j++) {
      const float ls = (float)l * scaling;
      ang[(int64_t)l * nr + j] = ls * powf(theta, (-2.f * (float)j) / (float)t_real);
    }
  return nr;
}

/* src/model/blocks.cpp:112-199 sdpa (non-causal), as the reference build's
 * AVX2 path evaluates it: per head and query row i, s[j] = fl(dot * scale)
 * with dot a serial fused multiply-add chain over d (scale = 1/sqrtf(hd));
 * mx = max_j s[j]; p[j] = expf(s[j] - mx); sum = serial float sum of p;
 * p[j] = fl(p[j] * fl(1/sum)); out[i, d] = serial fma chain over j of
 * p[j] * v[j, d]. Rows of stride ldq / ldk / ldv / ldo floats; head h uses
 * columns h*hd .. h*hd+hd-1. p: scratch of Lk floats. */
void orc_sdpa(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v, int64_t ldv,
              float* out, int64_t ldo, int64_t Lq, int64_t Lk, int heads, int hd, float* p) {
  const float scale = 1.f / sqrtf((float)hd);
  for (int h = 0; h < heads; h++)
    for (int64_t i = 0; i < Lq; i++) {
      const float* qi = q + i * ldq + (int64_t)h * hd;
      float mx = -INFINITY;
      for (int64_t j = 0; j < Lk; j++) {
        const float* kj = k + j * ldk + (int64_t)h * hd;
        float acc = 0.f;
        for (int d = 0; d < hd; d++) acc = fmaf(qi[d], kj[d], acc);
        p[j] = acc * scale;
        mx = p[j] > mx ? p[j] : mx;
      }
      float sum = 0.f;
      for (int64_t j = 0; j < Lk; j++) {
        p[j] = expf(p[j] - mx);
        sum = sum + p[j];
      }
      const float inv = 1.f / sum;
      for (int64_t j = 0; j < Lk; j++) p[j] = p[j] * inv;
      float* o = out + i * ldo + (int64_t)h * hd;
      for (int d = 0; d < hd; d++) {
        float acc = 0.f;
        for (int64_t j = 0; j < Lk; j++) acc = fmaf(p[j], v[j * ldv + (int64_t)h * hd + d], acc);
        o[d] = acc;
      }
    }
}

/* src/model/ovi_dit.cpp:132-142 gelu_tanh_inplace (nn.GELU(approximate='tanh')).
 * Uses libm tanhf; not bit-reproducible across libms, so only tolerance
 * checks use it. */
void orc_gelu_tanh(float* x, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    float v = x[i];
    float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    x[i] = 0.5f * v * (1.f + tanhf(u));
  }
}

/* src/core/tensor.cpp:63-78 quantize_rowwise: sc = fl(mx/127), sc==0 -> 1,
 * q = (int8) lround(w / sc)  (half away from zero, no clamp). */
void orc_quantize_rowwise(const float* W, int64_t N, int64_t K, int8_t* q, float* s) {
  for (int64_t i = 0; i < N; i++) {
    float mx = 0.f;
    for (int64_t k = 0; k < K; k++) {
      float a = fabsf(W[i * K + k]);
      mx = (mx < a) ? a : mx;
    }
    float sc = mx / 127.f;
    if (sc == 0.f) sc = 1.f;
    s[i] = sc;
    for (int64_t k = 0; k < K; k++) {
      float v = W[i * K + k] / sc;
      q[i * K + k] = (int8_t)lroundf(v);
    }
  }
}

/* tools/quantize/pack_sdcpp.py:45-51 quant_rows (numpy float32 semantics):
 *   amax = max|x| per row; safe = amax>0 ? amax : 1
 *   q = clip(rint(x * fl32(127/safe)), -127, 127)   (rint: ties to even)
 *   scale = fl32(amax / 127)                        (0 for an all-zero row) */
void orc_quant_rows(const float* W, int64_t N, int64_t K, int8_t* q, float* s) {
  for (int64_t i = 0; i < N; i++) {
    float amax = 0.f;
    for (int64_t k = 0; k < K; k++) {
      float a = fabsf(W[i * K + k]);
      amax = (amax < a) ? a : amax;
    }
    float safe = amax > 0.f ? amax : 1.f;
    float mul = 127.f / safe;
    for (int64_t k = 0; k < K; k++) {
      float v = rintf(W[i * K + k] * mul);
      if (v < -127.f) v = -127.f;
      if (v > 127.f) v = 127.f;
      q[i * K + k] = (int8_t)v;
    }
    s[i] = amax / 127.f;
  }
}

/* src/core/tensor.cpp:125-132 randu: xorshift64, values in [-1, 1]. */
void orc_randu(float* x, int64_t n, uint64_t seed) {
  uint64_t s = seed ? seed : 0x9e3779b97f4a7c15ull;
  for (int64_t i = 0; i < n; i++) {
    s ^= s << 13; s ^= s >> 7; s ^= s << 17;
    x[i] = (float)((int32_t)(s >> 40) % 20001 - 10000) / 10000.f;
  }
}

/* src/pipeline/gen.cpp:88-105 randn: splitmix64 + Box-Muller in double. */
void orc_randn(float* x, int64_t n, uint64_t seed) {
  uint64_t s = seed + 0x9E3779B97F4A7C15ull;
  for (int64_t i = 0; i < n; i += 2) {
    uint64_t z;
    z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    uint64_t n1 = z ^ (z >> 31);
    z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    uint64_t n2 = z ^ (z >> 31);
    const double u1 = ((double)(n1 >> 11) + 1.0) / 9007199254740993.0;
    const double u2 = (double)(n2 >> 11) / 9007199254740992.0;
    const double r = sqrt(-2.0 * log(u1));
    x[i] = (float)(r * cos(6.283185307179586 * u2));
    if (i + 1 < n) x[i + 1] = (float)(r * sin(6.283185307179586 * u2));
  }
}
