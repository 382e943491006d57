// Runs the reference's own OviDit::forward (src/model/ovi_dit.cpp:600-768) at
// OviDitCfg::test() (ovi_dit.cpp:336-342) on a .sdcpp pack and fixed inputs,
// as tests/test_ovit8.cpp:83-125 does, and writes both outputs. Written
// against the reference's headers; oracle/Makefile builds it from the
// reference's sources where they lie, twice:
//   _ref/ref_forward_cpu: with the reference's src/core/qgemm.cpp;
//   _ref/ref_forward_gpu: without it, linked to libsd_qgemm.so (sd::qgemm on
//     the MI355X, -DREF_FORWARD_GPU): the reference's link line with
//     -lsd_qgemm -lsdq in place of qgemm.cpp.
// Every other step (patch embeds, norms, attention, GELU, the bias pass of
// mlin) is the same compiled reference code in both.
//
// usage: ref_forward <pack.sdcpp> <in_dir> <out_dir> <iters>
//   in_dir/dims.txt: "F H W La Lc t"; video.bin [48,F,H,W], audio.bin [La,20],
//   vctx.bin, actx.bin [Lc,512], all float32.
//   out_dir/out_video.bin, out_audio.bin; one "forward_ms <i> <ms>" line per
//   iteration on stdout.
#include "model/ovi_dit.h"

#include <chrono>
#include <cstdio>
#include <stdexcept>
#include <string>

#ifdef REF_FORWARD_GPU
#include "sdq.h"
#endif

using sd::DType;
using sd::Tensor;

static Tensor read_f32(const std::string& path, std::vector<int64_t> shape) {
  Tensor t(shape, DType::F32);
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) throw std::runtime_error("cannot open " + path);
  const size_t got = std::fread(t.data, 1, t.nbytes, f);
  std::fclose(f);
  if (got != t.nbytes) throw std::runtime_error("short read " + path);
  return t;
}

static void write_f32(const std::string& path, const Tensor& t) {
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(t.data, 1, t.nbytes, f) != t.nbytes)
    throw std::runtime_error("cannot write " + path);
  std::fclose(f);
}

int main(int argc, char** argv) {
  if (argc != 5) {
    std::fprintf(stderr, "usage: ref_forward <pack> <in_dir> <out_dir> <iters>\n");
    return 2;
  }
  try {
#ifdef REF_FORWARD_GPU
    if (sdq_init(0) != SDQ_OK) throw std::runtime_error(sdq_last_error());
#endif
    const std::string in = argv[2], out = argv[3];
    const int iters = std::atoi(argv[4]);
    long long F, H, W, La, Lc;
    float t;
    FILE* d = std::fopen((in + "/dims.txt").c_str(), "r");
    if (!d || std::fscanf(d, "%lld %lld %lld %lld %lld %f", &F, &H, &W, &La, &Lc, &t) != 6)
      throw std::runtime_error("bad dims.txt");
    std::fclose(d);
    Tensor nv = read_f32(in + "/video.bin", {48, F, H, W});
    Tensor na = read_f32(in + "/audio.bin", {La, 20});
    Tensor vctx = read_f32(in + "/vctx.bin", {Lc, 512});
    Tensor actx = read_f32(in + "/actx.bin", {Lc, 512});
    sd::ovi::OviDit dit;
    dit.init(sd::ovi::OviDitCfg::test());
    dit.load_quantized_pack(argv[1]);
    std::printf("use_int8 %d\n", dit.use_int8 ? 1 : 0);
    Tensor ov, oa;
    for (int i = 0; i < iters; i++) {
      const auto t0 = std::chrono::steady_clock::now();
      dit.forward(nv, na, t, vctx, actx, ov, oa);
      const double ms =
          std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
      std::printf("forward_ms %d %.3f\n", i, ms);
    }
    write_f32(out + "/out_video.bin", ov);
    write_f32(out + "/out_audio.bin", oa);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "ref_forward: %s\n", e.what());
    return 1;
  }
  return 0;
}
