// PackIndex and load_sdcpp: see sd/pack.h.
//
// The tensor table is read front to back through a small buffer of file
// reads (a 12 GB pack's table is a few hundred KB; nothing else is touched),
// and every entry is resolved to absolute file offsets. The mapping is made
// only by load_sdcpp, whose views the reference's callers expect; uploads
// that read the tensors with sequential reads use the index alone.
//
// The checks and their messages are the reference loader's error contract
// (src/serde/sdcpp.cpp:27-29, 47-105): callers and tests match on them.
#include "sd/pack.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace sd {
namespace {

[[noreturn]] void fail(const std::string& m) { throw std::runtime_error("sdcpp: " + m); }

constexpr int64_t kMaxNumel = int64_t(1) << 40;  // the reference's size guard
constexpr uint32_t kMaxDims = 8;

// Sequential reader of the table: refills a 1 MB window with pread; `off` is
// the absolute file offset of the next unread byte.
class TableStream {
 public:
  TableStream(int fd, uint64_t size) : fd_(fd), size_(size), buf_(1 << 20) {}
  void take(void* dst, size_t n) {
    if (size_ - off_ < n) fail("truncated file");
    char* d = static_cast<char*>(dst);
    while (n) {
      if (pos_ == len_) refill();
      const size_t k = std::min(n, len_ - pos_);
      std::memcpy(d, buf_.data() + pos_, k);
      pos_ += k;
      off_ += k;
      d += k;
      n -= k;
    }
  }
  template <typename T> T num() {
    T v;
    take(&v, sizeof v);
    return v;
  }
  uint64_t offset() const { return off_; }

 private:
  void refill() {
    const size_t want = (size_t)std::min<uint64_t>(buf_.size(), size_ - off_);
    ssize_t got;
    do {
      got = ::pread(fd_, buf_.data(), want, (off_t)off_);
    } while (got < 0 && errno == EINTR);
    if (got <= 0) fail("truncated file");
    len_ = (size_t)got;
    pos_ = 0;
  }
  int fd_;
  uint64_t size_, off_ = 0;
  std::vector<char> buf_;
  size_t pos_ = 0, len_ = 0;
};

struct Fd {
  int v = -1;
  ~Fd() {
    if (v >= 0) ::close(v);
  }
};

}  // namespace

PackIndex PackIndex::read(const std::string& path) {
  Fd fd;
  fd.v = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd.v < 0) fail("cannot open " + path);
  struct stat st;
  if (::fstat(fd.v, &st) != 0 || st.st_size < 16) fail("truncated file " + path);
  PackIndex ix;
  ix.path_ = path;
  ix.size_ = (uint64_t)st.st_size;
  TableStream in(fd.v, ix.size_);
  char magic[4];
  in.take(magic, 4);
  if (std::memcmp(magic, "SDCP", 4) != 0) fail("bad magic");
  if (in.num<uint32_t>() != 1) fail("unsupported version");
  const uint32_t count = in.num<uint32_t>();

  // First pass over the table: shapes and data-relative offsets.
  struct Row {
    std::string name;
    PackEntry e;
    uint64_t rel;
  };
  std::vector<Row> rows;
  rows.reserve(std::min<uint32_t>(count, 1u << 16));
  for (uint32_t i = 0; i < count; i++) {
    Row r;
    r.e.position = i;
    const uint32_t name_len = in.num<uint32_t>();
    r.name.resize(name_len);
    in.take(r.name.data(), name_len);
    const uint8_t code = in.num<uint8_t>();
    if (code > 1) fail("bad dtype code");
    r.e.kind = code == 0 ? PackEntry::kInt8Rows : PackEntry::kF32;
    const uint32_t nd = in.num<uint32_t>();
    if (nd > kMaxDims) fail("ndim too large");
    int64_t numel = 1;
    r.e.dims.resize(nd);
    for (int64_t& d : r.e.dims) {
      d = (int64_t)in.num<uint64_t>();
      if (d < 0) fail("negative dim");
      if (d != 0 && numel > kMaxNumel / d) fail("tensor too large");
      numel *= d;
    }
    r.e.numel = numel;
    r.rel = in.num<uint64_t>();
    if (r.e.kind == PackEntry::kInt8Rows) {
      if (nd == 0 || r.e.dims.back() < 1) fail("quantized tensor needs a last dim");
      r.e.rows = numel / r.e.dims.back();
      r.e.bytes = (uint64_t)numel + (uint64_t)r.e.rows * 4;
    } else {
      r.e.bytes = (uint64_t)numel * 4;
    }
    rows.push_back(std::move(r));
  }
  // The data region is the rest of the file.
  const uint64_t base = in.offset(), avail = ix.size_ - base;
  for (const Row& r : rows)
    if (r.rel > avail || r.e.bytes > avail - r.rel) fail("data out of bounds");
  ix.table_.reserve(rows.size());
  for (Row& r : rows) {
    r.e.data = base + r.rel;
    r.e.scale = r.e.kind == PackEntry::kInt8Rows ? r.e.data + (uint64_t)r.e.numel : 0;
    if (r.e.kind == PackEntry::kInt8Rows)
      ix.int8_first_.emplace(r.name, (uint32_t)ix.table_.size());
    if (ix.map_.emplace(r.name, r.e).second)  // first of a repeated name wins
      ix.order_.push_back(r.name);
    ix.table_.emplace_back(std::move(r.name), std::move(r.e));
  }
  return ix;
}

const PackEntry* PackIndex::find(const std::string& name) const {
  auto it = map_.find(name);
  return it == map_.end() ? nullptr : &it->second;
}

const PackEntry* PackIndex::f32_view(const std::string& name, bool* scale_of_int8) const {
  const PackEntry* raw = find(name);
  const PackEntry* q = nullptr;
  const std::string suffix = ".scale";
  if (name.size() > suffix.size() &&
      name.compare(name.size() - suffix.size(), suffix.size(), suffix) == 0) {
    auto it = int8_first_.find(name.substr(0, name.size() - suffix.size()));
    if (it != int8_first_.end()) q = &table_[it->second].second;
  }
  // load_sdcpp emplaces views in table order: the earlier entry owns the name
  const bool use_q = q && (!raw || q->position < raw->position);
  if (scale_of_int8) *scale_of_int8 = use_q;
  if (use_q) return q;
  return raw && raw->kind == PackEntry::kF32 ? raw : nullptr;
}

std::vector<float> PackIndex::read_f32(const PackEntry& e, bool scales) const {
  const size_t n = (size_t)(scales ? e.rows : e.numel);
  const uint64_t off = scales ? e.scale : e.data;
  std::vector<float> v(n);
  Fd fd;
  fd.v = ::open(path_.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd.v < 0) fail("cannot open " + path_);
  char* d = reinterpret_cast<char*>(v.data());
  size_t left = n * 4;
  uint64_t o = off;
  while (left) {
    const ssize_t got = ::pread(fd.v, d, left, (off_t)o);
    if (got < 0 && errno == EINTR) continue;
    if (got <= 0) fail("truncated file");
    d += got;
    o += (uint64_t)got;
    left -= (size_t)got;
  }
  return v;
}

std::unordered_map<std::string, Tensor> load_sdcpp(const std::string& path,
                                                   std::shared_ptr<void>& owner) {
  const PackIndex ix = PackIndex::read(path);
  Fd fd;
  fd.v = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd.v < 0) fail("cannot open " + path);
  const size_t size = (size_t)ix.file_size();
  void* map = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd.v, 0);
  if (map == MAP_FAILED) fail("mmap failed " + path);
  owner = std::shared_ptr<void>(map, [size](void* p) { ::munmap(p, size); });
  char* at = static_cast<char*>(map);
  std::unordered_map<std::string, Tensor> views;
  views.reserve(ix.entries().size() * 2);
  auto view = [&](uint64_t off, std::vector<int64_t> shape, DType dt, size_t bytes) {
    Tensor t;
    t.shape = std::move(shape);
    t.dtype = dt;
    t.data = at + off;
    t.nbytes = bytes;
    t.owning = false;
    return t;
  };
  for (const auto& [name, e] : ix.table()) {  // table order: the first view of a name wins
    if (e.kind == PackEntry::kInt8Rows) {
      views.emplace(name, view(e.data, e.dims, DType::I8, (size_t)e.numel));
      views.emplace(name + ".scale", view(e.scale, {e.rows}, DType::F32, (size_t)e.rows * 4));
    } else {
      views.emplace(name, view(e.data, e.dims, DType::F32, (size_t)e.bytes));
    }
  }
  return views;
}

}  // namespace sd
