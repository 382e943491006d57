// .sdcpp v1 loader, same contract as the reference's src/serde/sdcpp.h:
// quantized tensors appear as an I8 view under `name` (original shape) plus
// an F32 per-row scale view under `name.scale`; raw tensors as one F32 view.
// `owner` keeps the mmap alive. Throws std::runtime_error("sdcpp: …") on a
// missing file, bad magic/version/dtype, truncation or out-of-bounds data.
#pragma once
#include <memory>
#include <string>
#include <unordered_map>

#include "sd/tensor.h"

namespace sd {

std::unordered_map<std::string, Tensor> load_sdcpp(const std::string& path,
                                                   std::shared_ptr<void>& owner);

}  // namespace sd
