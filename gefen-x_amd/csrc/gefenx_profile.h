// gefenx_profile.h -- launch bracketing for the optional kernel timing.
#pragma once
#include <hip/hip_runtime.h>

namespace gx {
// Returns a handle (or -1 when timing is off); pair with prof_end.
int prof_begin(int kind, double algo_bytes, double algo_flops, hipStream_t s);
void prof_end(int handle, hipStream_t s);
}  // namespace gx
