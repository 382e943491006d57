// The reference's loader header name (src/serde/sdcpp.h): load_sdcpp with the
// same contract, declared with the pack index in sd/pack.h.
#pragma once
#include "sd/pack.h"
