// citlali/compute/hip/hip_check.h -- turns a C-ABI status into citlali::Error.
//
// Replaces the reference's CITLALI_CUDA_CHECK (cuda_utils.h:17-26).  The
// C ABI already formats HIP failures as
// "HIP error at <file>:<line> for <expr>: <message>"; argument errors carry
// the library's validation message.  Either is rethrown unchanged.
#pragma once

#include "citlali/common.h"
#include "citlali_hip.h"

#include <string>

namespace citlali::compute {

inline void check_status(int status, const char* expression) {
    if (status == CITLALI_OK) return;
    const char* msg = citlali_hip_last_error();
    throw Error((msg && *msg) ? std::string(msg) : std::string("citlali_hip call failed: ") + expression);
}

}  // namespace citlali::compute

#define CITLALI_HIP_CHECK(expr) ::citlali::compute::check_status((expr), #expr)
