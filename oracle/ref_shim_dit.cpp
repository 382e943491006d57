// CPU ORACLE — test infrastructure only (never linked by the shipped library).
//
// C wrappers around the REFERENCE's DiT glue that sits next to the int8
// Linears: blk::layernorm (src/model/blocks.cpp:18-43), mod_rows
// (src/model/ovi_dit.cpp:161-172), sd::rmsnorm (src/core/tensor.cpp:112-123),
// blk::apply_rope and the rope angle tables (src/model/blocks.cpp:46-100). mod_rows has internal linkage, so this
// translation unit compiles the reference's ovi_dit.cpp itself, in place
// (oracle/Makefile passes -I<reference>/src); only the wrappers are ours.
#include "model/ovi_dit.cpp"

namespace {

sd::Tensor fview(const float* p, std::initializer_list<int64_t> shape) {
  sd::Tensor t;
  t.shape = shape;
  t.dtype = sd::DType::F32;
  t.data = const_cast<float*>(p);
  int64_t n = 1;
  for (auto d : shape) n *= d;
  t.nbytes = (size_t)n * 4;
  t.owning = false;
  return t;
}

}  // namespace

extern "C" {

// blk::layernorm(x, y, w, b, eps) on caller buffers [M,N] (w, b nullable).
int sdref_layernorm(const float* x, int64_t M, int64_t N, float eps, const float* w,
                    const float* b, float* y) {
  try {
    sd::Tensor out, tw, tb;
    if (w) tw = fview(w, {N});
    if (b) tb = fview(b, {N});
    sd::blk::layernorm(fview(x, {M, N}), out, w ? &tw : nullptr, b ? &tb : nullptr, eps);
    std::memcpy(y, out.data, (size_t)(M * N) * 4);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// mod_rows(x, shift, scale, y): y = x*(1+scale)+shift, [L,C] with [C] rows.
int sdref_mod_rows(const float* x, const float* shift, const float* scale, int64_t L, int64_t C,
                   float* y) {
  try {
    sd::Tensor out;
    sd::ovi::mod_rows(fview(x, {L, C}), fview(shift, {C}), fview(scale, {C}), out);
    std::memcpy(y, out.data, (size_t)(L * C) * 4);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// sd::rmsnorm(x, w, eps) in place on caller buffers [M,N] (tensor.cpp:112).
int sdref_rmsnorm(float* x, int64_t M, int64_t N, const float* w, float eps) {
  try {
    sd::Tensor t = fview(x, {M, N});
    sd::rmsnorm(t, fview(w, {N}), eps);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// blk::apply_rope(x, {ang, nr}, heads) in place on [L,C] (blocks.cpp:86).
int sdref_apply_rope(float* x, int64_t L, int64_t C, const float* ang, int nr, int heads) {
  try {
    sd::Tensor t = fview(x, {L, C});
    sd::blk::RopeFreqs f;
    f.n_rot = nr;
    f.ang = fview(ang, {L, nr});
    sd::blk::apply_rope(t, f, heads);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// blk::rope_freqs_3d / rope_freqs_1d angle tables (blocks.cpp:46-84) into
// ang (room for rows * n_rot floats); returns n_rot, or -1.
int sdref_rope_freqs_3d(int T, int H, int W, int hd, float theta, float* ang) {
  try {
    sd::blk::RopeFreqs f = sd::blk::rope_freqs_3d(T, H, W, hd, theta);
    std::memcpy(ang, f.ang.data, (size_t)T * H * W * f.n_rot * 4);
    return f.n_rot;
  } catch (const std::exception&) {
    return -1;
  }
}

int sdref_rope_freqs_1d(int L, int hd, float theta, float scaling, float* ang) {
  try {
    sd::blk::RopeFreqs f = sd::blk::rope_freqs_1d(L, hd, theta, scaling);
    std::memcpy(ang, f.ang.data, (size_t)L * f.n_rot * 4);
    return f.n_rot;
  } catch (const std::exception&) {
    return -1;
  }
}

// blk::sdpa(q, k, v, heads, out) (blocks.cpp:112-199) on contiguous [L, C].
int sdref_sdpa(const float* q, const float* k, const float* v, int64_t Lq, int64_t Lk, int64_t C,
               int heads, float* out) {
  try {
    sd::Tensor o;
    sd::blk::sdpa(fview(q, {Lq, C}), fview(k, {Lk, C}), fview(v, {Lk, C}), heads, o, false);
    std::memcpy(out, o.data, (size_t)(Lq * C) * 4);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

}  // extern "C"
