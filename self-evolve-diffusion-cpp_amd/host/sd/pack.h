// .sdcpp v1 packs on the host: an index of the tensor table, read with plain
// file reads (no mapping), and the loader contract of the reference built on
// it.
//
// Format (src/serde/sdcpp.cpp:1-8, written by tools/quantize/pack_sdcpp.py):
//   "SDCP" | u32 version = 1 | u32 count
//   count x { u32 name_len | name | u8 code (0 = int8 rowwise, 1 = f32)
//             | u32 ndim | i64 dims[ndim] | u64 offset into the data region }
//   data region (right after the table): code 0 -> i8[numel] then f32[rows]
//   (rows = numel / dims[-1]); code 1 -> f32[numel]. Little-endian, no padding.
//
// The index keeps absolute file offsets, so a reader can move a tensor's
// bytes with large sequential reads (PackReader, and the library's file
// upload sdq_weight_upload_file) instead of page-faulting through a mapping.
#pragma once
#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "sd/tensor.h"

namespace sd {

struct PackEntry {
  enum Kind : uint8_t { kInt8Rows = 0, kF32 = 1 } kind = kF32;
  std::vector<int64_t> dims;
  int64_t numel = 0;
  int64_t rows = 0;       // kInt8Rows: numel / dims.back(), one f32 scale each
  uint64_t data = 0;      // absolute file offset of the int8 (or f32) data
  uint64_t scale = 0;     // kInt8Rows: absolute file offset of the scales
  uint64_t bytes = 0;     // all of the entry's bytes (data + scales)
  uint32_t position = 0;  // index in the tensor table
};

class PackIndex {
 public:
  // Reads and checks the tensor table; throws std::runtime_error("sdcpp: …")
  // with the reference loader's messages on a missing file, bad magic,
  // version or dtype code, truncation or data out of bounds.
  static PackIndex read(const std::string& path);
  const PackEntry* find(const std::string& name) const;
  const std::unordered_map<std::string, PackEntry>& entries() const { return map_; }
  // Names in table order (a repeated name is listed once, at its first entry).
  const std::vector<std::string>& order() const { return order_; }
  // Every entry in table order, repeated names included.
  const std::vector<std::pair<std::string, PackEntry>>& table() const { return table_; }
  uint64_t file_size() const { return size_; }
  // The view load_sdcpp gives `name`, when it is an F32 one: the first entry
  // called `name`, or the scales of the first int8 entry called `name` minus
  // ".scale", whichever comes first in the table (the loader emplaces views in
  // table order and the first view of a name wins); nullptr when neither
  // exists or the winner is an int8 tensor. *scale_of_int8 tells which.
  const PackEntry* f32_view(const std::string& name, bool* scale_of_int8) const;
  // Reads a raw F32 entry's values (or an int8 entry's scales) from the file.
  std::vector<float> read_f32(const PackEntry& e, bool scales) const;
  const std::string& path() const { return path_; }

 private:
  std::string path_;
  uint64_t size_ = 0;
  std::unordered_map<std::string, PackEntry> map_;       // first entry of each name
  std::unordered_map<std::string, uint32_t> int8_first_;  // name -> table_ index
  std::vector<std::string> order_;
  std::vector<std::pair<std::string, PackEntry>> table_;
};

// The reference's loader contract (src/serde/sdcpp.h:18-19): the file mapped
// read-only; quantized tensors as an I8 view under `name` (original shape)
// plus an F32 per-row scale view under `name.scale`, raw tensors as one F32
// view; `owner` keeps the mapping alive.
std::unordered_map<std::string, Tensor> load_sdcpp(const std::string& path,
                                                   std::shared_ptr<void>& owner);

}  // namespace sd
