// Internal hooks of the opt-in per-stage timing (dcn2_profile.cpp); no-ops
// unless dcn2_profile_enable(1) was called on this thread.
#pragma once

#include <hip/hip_runtime.h>

namespace dcn2 {
void prof_begin(int stage, hipStream_t s);
void prof_end(int stage, hipStream_t s);
}  // namespace dcn2
