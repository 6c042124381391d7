// Declarations shared between the library's translation units (not ABI).
#pragma once

#include "rfsn_common.h"

namespace rfsn {

int launch_merge(const float* partial, int64_t bh, int splits, int D, void* out, hipStream_t s);

}  // namespace rfsn
