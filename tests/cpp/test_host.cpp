// Driver for the C++17 host mirror (sd::Tensor, sd::qgemm, sd::load_sdcpp,
// sd::gpu::QLinear), run by tests/test_host_api.py. Inputs and outputs are
// raw little-endian arrays so the Python side can compare them with the
// oracle. Subcommands:
//   sdcpp <pack>                    list entries: name code ndim dims... off soff
//   sdcpp_err <pack>                exit 0 iff load_sdcpp throws (prints what())
//   qgemm M K N A.bin Bq.bin bs.bin out.bin
//   qgemm_threads M K N A.bin Bq.bin bs.bin out.bin threads reps
//   linear <pack> <base> in out M mode x.bin gate.bin res.bin out.bin
//          mode: mlin | gelu | gated | add   (gate/res ignored when unused)
//   linear_err <pack> <base> in out  exit 0 iff qlinear_from_pack throws
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "sd/pack.h"
#include "sd/qlinear.h"
#include "sd/tensor.h"

using namespace sd;

static std::vector<char> read_file(const std::string& p) {
  std::ifstream f(p, std::ios::binary);
  if (!f) throw std::runtime_error("cannot read " + p);
  return std::vector<char>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

static void write_file(const std::string& p, const void* d, size_t n) {
  std::ofstream f(p, std::ios::binary);
  f.write(static_cast<const char*>(d), (std::streamsize)n);
  if (!f) throw std::runtime_error("cannot write " + p);
}

static Tensor load_tensor(const std::string& p, std::vector<int64_t> shape, DType dt) {
  Tensor t(shape, dt);
  std::vector<char> b = read_file(p);
  if (b.size() != t.nbytes) throw std::runtime_error("size mismatch for " + p);
  std::memcpy(t.data, b.data(), b.size());
  return t;
}

static int cmd_sdcpp(const std::string& path) {
  std::shared_ptr<void> owner;
  auto m = load_sdcpp(path, owner);
  const char* base = static_cast<const char*>(owner.get());
  for (auto& kv : m) {
    const Tensor& t = kv.second;
    std::printf("%s %d %zu", kv.first.c_str(), (int)t.dtype, t.shape.size());
    for (int64_t d : t.shape) std::printf(" %lld", (long long)d);
    std::printf(" %lld\n", (long long)(static_cast<const char*>(t.data) - base));
  }
  return 0;
}

// The F32 view PackIndex::f32_view resolves for `name`: its data offset, and
// whether it is an int8 entry's scales.
static int cmd_f32view(const std::string& path, const std::string& name) {
  const PackIndex ix = PackIndex::read(path);
  bool scales = false;
  const PackEntry* e = ix.f32_view(name, &scales);
  if (!e)
    std::printf("none\n");
  else
    std::printf("%s %llu\n", scales ? "scales" : "f32",
                (unsigned long long)(scales ? e->scale : e->data));
  return 0;
}

static int cmd_sdcpp_err(const std::string& path) {
  try {
    std::shared_ptr<void> owner;
    load_sdcpp(path, owner);
  } catch (const std::runtime_error& e) {
    std::printf("%s\n", e.what());
    return 0;
  }
  std::printf("no throw\n");
  return 1;
}

// `threads` threads each call sd::qgemm `reps` times on the same weights while
// another thread keeps clearing the weight cache, so device copies are
// dropped from the cache while calls still use them. Every result must equal
// the first; that one is written for the oracle comparison.
static int cmd_qgemm_threads(char** argv) {
  gpu::check(sdq_init(0), "sdq_init");
  const int64_t M = std::atoll(argv[2]), K = std::atoll(argv[3]), N = std::atoll(argv[4]);
  const int threads = std::atoi(argv[9]), reps = std::atoi(argv[10]);
  const Tensor A = load_tensor(argv[5], {M, K}, DType::F32);
  const Tensor Bq = load_tensor(argv[6], {N, K}, DType::I8);
  const Tensor bs = load_tensor(argv[7], {N}, DType::F32);
  Tensor first;
  qgemm(A, Bq, bs, first);
  std::atomic<int> bad{0}, calls{0}, clears{0};
  std::atomic<bool> done{false};
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; t++)
    pool.emplace_back([&] {
      try {
        for (int r = 0; r < reps; r++) {
          Tensor out;
          qgemm(A, Bq, bs, out);
          calls++;
          if (std::memcmp(out.data, first.data, first.nbytes) != 0) bad++;
        }
      } catch (const std::exception& e) {
        std::fprintf(stderr, "worker: %s\n", e.what());
        bad++;
      }
    });
  std::thread clearer([&] {
    while (!done.load()) {
      qgemm_cache_clear();
      clears++;
      std::this_thread::yield();
    }
  });
  for (auto& th : pool) th.join();
  done = true;
  clearer.join();
  qgemm_cache_clear();
  std::printf("calls %d mismatches %d clears %d cache entries %zu\n", calls.load(), bad.load(),
              clears.load(), qgemm_cache_size());
  write_file(argv[8], first.data, first.nbytes);
  return bad.load() == 0 ? 0 : 1;
}

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: test_host <cmd> ...\n");
    return 2;
  }
  const std::string cmd = argv[1];
  try {
    if (cmd == "sdcpp" && argc == 3) return cmd_sdcpp(argv[2]);
    if (cmd == "sdcpp_err" && argc == 3) return cmd_sdcpp_err(argv[2]);
    if (cmd == "f32view" && argc == 4) return cmd_f32view(argv[2], argv[3]);
    if (cmd == "qgemm" && argc == 9) {
      gpu::check(sdq_init(0), "sdq_init");
      const int64_t M = std::atoll(argv[2]), K = std::atoll(argv[3]), N = std::atoll(argv[4]);
      Tensor A = load_tensor(argv[5], {M, K}, DType::F32);
      Tensor Bq = load_tensor(argv[6], {N, K}, DType::I8);
      Tensor bs = load_tensor(argv[7], {N}, DType::F32);
      Tensor out;
      qgemm(A, Bq, bs, out);
      // second call hits the weight cache
      Tensor out2;
      qgemm(A, Bq, bs, out2);
      if (std::memcmp(out.data, out2.data, out.nbytes) != 0) {
        std::fprintf(stderr, "cached call differs\n");
        return 1;
      }
      std::printf("cache entries %zu\n", qgemm_cache_size());
      // new contents at the same addresses (a pack mapped again in place):
      // the cached device copy must be replaced, not reused
      int8_t* q = Bq.ptr<int8_t>();
      float* s = bs.ptr<float>();
      for (int64_t i = 0; i < N * K; i++) q[i] = (int8_t)(-q[i]);
      for (int64_t j = 0; j < N; j++) s[j] = 2.f * s[j];
      Tensor out3;
      qgemm(A, Bq, bs, out3);
      std::printf("cache entries after rewrite %zu\n", qgemm_cache_size());
      qgemm_cache_clear();
      write_file(argv[8], out.data, out.nbytes);
      write_file(std::string(argv[8]) + ".rewritten", out3.data, out3.nbytes);
      return 0;
    }
    if (cmd == "qgemm_threads" && argc == 11) return cmd_qgemm_threads(argv);
    if (cmd == "linear" && argc == 12) {
      gpu::check(sdq_init(0), "sdq_init");
      std::shared_ptr<void> owner;
      auto pack = load_sdcpp(argv[2], owner);
      const std::string base = argv[3];
      const int64_t in = std::atoll(argv[4]), out = std::atoll(argv[5]), M = std::atoll(argv[6]);
      const std::string mode = argv[7];
      gpu::QLinear lin = gpu::qlinear_from_pack(pack, base, in, out);
      Tensor x = load_tensor(argv[8], {M, in}, DType::F32);
      Tensor y;
      if (mode == "mlin") {
        lin.mlin(x, y);
      } else if (mode == "gelu") {
        lin.mlin_gelu(x, y);
      } else if (mode == "gated") {
        Tensor g = load_tensor(argv[9], {out}, DType::F32);
        y = load_tensor(argv[10], {M, out}, DType::F32);
        lin.mlin_gated_add(x, g, y);
      } else if (mode == "add") {
        y = load_tensor(argv[10], {M, out}, DType::F32);
        lin.mlin_add(x, y);
      } else {
        throw std::runtime_error("bad mode " + mode);
      }
      write_file(argv[11], y.data, y.nbytes);
      return 0;
    }
    // mlin for either weight dtype (sd::gpu::linear_from_pack: I8 or F32)
    if (cmd == "mlin_any" && argc == 9) {
      gpu::check(sdq_init(0), "sdq_init");
      std::shared_ptr<void> owner;
      auto pack = load_sdcpp(argv[2], owner);
      const int64_t in = std::atoll(argv[4]), out = std::atoll(argv[5]), M = std::atoll(argv[6]);
      gpu::Linear lin = gpu::linear_from_pack(pack, argv[3], in, out);
      std::printf("int8 %d\n", lin.is_int8() ? 1 : 0);
      Tensor x = load_tensor(argv[7], {M, in}, DType::F32);
      Tensor y;
      lin.mlin(x, y);
      write_file(argv[8], y.data, y.nbytes);
      return 0;
    }
    if (cmd == "mlin_any_err" && argc == 6) {
      std::shared_ptr<void> owner;
      auto pack = load_sdcpp(argv[2], owner);
      try {
        gpu::Linear lin = gpu::linear_from_pack(pack, argv[3], std::atoll(argv[4]),
                                                std::atoll(argv[5]));
      } catch (const std::runtime_error& e) {
        std::printf("%s\n", e.what());
        return 0;
      }
      std::printf("no throw\n");
      return 1;
    }
    if (cmd == "linear_err" && argc == 6) {
      std::shared_ptr<void> owner;
      auto pack = load_sdcpp(argv[2], owner);
      try {
        gpu::QLinear lin = gpu::qlinear_from_pack(pack, argv[3], std::atoll(argv[4]),
                                                  std::atoll(argv[5]));
      } catch (const std::runtime_error& e) {
        std::printf("%s\n", e.what());
        return 0;
      }
      std::printf("no throw\n");
      return 1;
    }
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 3;
  }
  std::fprintf(stderr, "bad arguments for %s\n", cmd.c_str());
  return 2;
}
