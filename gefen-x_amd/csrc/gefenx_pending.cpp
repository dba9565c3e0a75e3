// gefenx_pending.cpp -- entry points declared in gefenx.h whose kernels are
// not built yet.  Each returns GEFENX_EINVAL with a clear message, so callers
// see a ValueError instead of a missing symbol.
#include "gefenx_internal.h"
#include "../../include/gefenx.h"

using gx::set_error;

extern "C" {

int gefenx_quantized_momentum_update(const void*, int, int64_t, int64_t, uint8_t*, float*,
                                     const void*, void*, double, int, int64_t, const int64_t*,
                                     int, void*, size_t, void*) {
    return set_error(GEFENX_EINVAL, "gefenx_quantized_momentum_update: not available in this build");
}

size_t gefenx_ns_workspace_bytes(int64_t, int64_t, int64_t) { return 0; }

int gefenx_newton_schulz(void*, int64_t, int64_t, int64_t, const float*, const float*,
                         const float*, int, float, void*, size_t, void*) {
    return set_error(GEFENX_EINVAL, "gefenx_newton_schulz: not available in this build");
}

}  // extern "C"
