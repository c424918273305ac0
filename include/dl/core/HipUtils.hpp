#pragma once
// HIP runtime error -> std::runtime_error("<action>: <HIP message>"), the
// convention of the reference's dl::cuda::check (src/core/CudaUtils.cpp:8-13).
// Internal to the library; the public dl.hpp does not include it.

#include <hip/hip_runtime_api.h>

namespace dl::hip {

void check(hipError_t status, const char* action);

// Throws std::runtime_error("<action>: <message>") for a non-zero fdl_status.
void check_fdl(int status, const char* action);

}  // namespace dl::hip
