// gefenx_internal.h -- declarations shared by the host translation units.
#pragma once

namespace gx {

// Record a thread-local error message and return `status`.
int set_error(int status, const char* fmt, ...);

float round_bf16(float x);
float round_f16(float x);

}  // namespace gx
