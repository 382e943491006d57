// .sdcpp v1 reader (host mirror of the reference's loader contract,
// src/serde/sdcpp.h; format in src/serde/sdcpp.cpp:1-8 and
// tools/quantize/pack_sdcpp.py:4-13):
//   "SDCP" | u32 version = 1 | u32 count
//   count x { u32 name_len | name | u8 code (0 = int8 rowwise, 1 = f32)
//             | u32 ndim | i64 dims[ndim] | u64 offset into the blob }
//   blob: code 0 -> i8[numel] then f32[rows] (rows = numel / dims[-1])
//         code 1 -> f32[numel]
// All little-endian, no alignment padding between blobs.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "sd/sdcpp.h"

namespace sd {
namespace {

[[noreturn]] void fail(const std::string& m) { throw std::runtime_error("sdcpp: " + m); }

class Cursor {
 public:
  Cursor(const uint8_t* b, const uint8_t* e) : p_(b), end_(e) {}
  void need(size_t n) const {
    if ((size_t)(end_ - p_) < n) fail("truncated file");
  }
  template <typename T> T get() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, p_, sizeof(T));
    p_ += sizeof(T);
    return v;
  }
  std::string str(size_t n) {
    need(n);
    std::string s(reinterpret_cast<const char*>(p_), n);
    p_ += n;
    return s;
  }
  const uint8_t* pos() const { return p_; }
  size_t left() const { return (size_t)(end_ - p_); }

 private:
  const uint8_t* p_;
  const uint8_t* end_;
};

struct Desc {
  std::string name;
  uint8_t code;
  std::vector<int64_t> dims;
  uint64_t off;
  int64_t numel, rows, blob;
};

constexpr int64_t kMaxNumel = int64_t(1) << 40;

}  // namespace

std::unordered_map<std::string, Tensor> load_sdcpp(const std::string& path,
                                                   std::shared_ptr<void>& owner) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) fail("cannot open " + path);
  struct stat st;
  if (::fstat(fd, &st) != 0 || st.st_size < 16) {
    ::close(fd);
    fail("truncated file " + path);
  }
  const size_t size = (size_t)st.st_size;
  void* base = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (base == MAP_FAILED) fail("mmap failed " + path);
  owner = std::shared_ptr<void>(base, [size](void* b) { ::munmap(b, size); });

  const uint8_t* b = static_cast<const uint8_t*>(base);
  Cursor c(b, b + size);
  if (c.str(4) != "SDCP") fail("bad magic");
  if (c.get<uint32_t>() != 1) fail("unsupported version");
  const uint32_t count = c.get<uint32_t>();

  std::vector<Desc> ds;
  ds.reserve(count < 65536 ? count : 65536);
  for (uint32_t i = 0; i < count; i++) {
    Desc d;
    const uint32_t nl = c.get<uint32_t>();
    d.name = c.str(nl);
    d.code = c.get<uint8_t>();
    if (d.code > 1) fail("bad dtype code");
    const uint32_t nd = c.get<uint32_t>();
    if (nd > 8) fail("ndim too large");
    int64_t numel = 1;
    for (uint32_t k = 0; k < nd; k++) {
      const int64_t x = (int64_t)c.get<uint64_t>();
      if (x < 0) fail("negative dim");
      if (x && numel > kMaxNumel / x) fail("tensor too large");
      numel *= x;
      d.dims.push_back(x);
    }
    d.numel = numel;
    d.off = c.get<uint64_t>();
    if (d.code == 0) {
      if (nd == 0 || d.dims.back() < 1) fail("quantized tensor needs a last dim");
      d.rows = numel / d.dims.back();
      d.blob = numel + d.rows * 4;
    } else {
      d.rows = 0;
      d.blob = numel * 4;
    }
    ds.push_back(std::move(d));
  }

  const uint8_t* blob = c.pos();
  const uint64_t avail = c.left();
  for (const Desc& d : ds)
    if (d.off > avail || (uint64_t)d.blob > avail - d.off) fail("data out of bounds");

  std::unordered_map<std::string, Tensor> out;
  for (const Desc& d : ds) {
    uint8_t* p = const_cast<uint8_t*>(blob + d.off);
    Tensor t;
    t.shape = d.dims;
    t.owning = false;
    t.data = p;
    if (d.code == 0) {
      t.dtype = DType::I8;
      t.nbytes = (size_t)d.numel;
      Tensor s;
      s.shape = {d.rows};
      s.dtype = DType::F32;
      s.data = p + d.numel;
      s.nbytes = (size_t)d.rows * 4;
      s.owning = false;
      out.emplace(d.name, std::move(t));
      out.emplace(d.name + ".scale", std::move(s));
    } else {
      t.dtype = DType::F32;
      t.nbytes = (size_t)d.blob;
      out.emplace(d.name, std::move(t));
    }
  }
  return out;
}

}  // namespace sd
