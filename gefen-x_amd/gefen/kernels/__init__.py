"""MI355X kernels of the Gefen optimizer step, reached through the C ABI in
include/gefenx.h (libgefenx.so, built for gfx950)."""
