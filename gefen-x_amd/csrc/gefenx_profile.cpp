// gefenx_profile.cpp -- optional HIP-event timing of every update-kernel launch.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "gefenx_internal.h"
#include "gefenx_profile.h"
#include "gefenx.h"

namespace gx {

namespace {
struct Rec {
    int kind;
    hipEvent_t e0, e1;
    double bytes, flops;
};
std::mutex g_mu;
bool g_enabled = false;
std::vector<Rec> g_open;       // launched, not yet read
std::vector<hipEvent_t> g_pool;

hipEvent_t take_event() {
    if (!g_pool.empty()) {
        hipEvent_t e = g_pool.back();
        g_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
}  // namespace

int prof_begin(int kind, double bytes, double flops, hipStream_t s) {
    if (!g_enabled) return -1;
    std::lock_guard<std::mutex> lk(g_mu);
    Rec r{kind, take_event(), take_event(), bytes, flops};
    if (!r.e0 || !r.e1) return -1;
    hipEventRecord(r.e0, s);
    g_open.push_back(r);
    return (int)g_open.size() - 1;
}

void prof_end(int handle, hipStream_t s) {
    if (handle < 0) return;
    std::lock_guard<std::mutex> lk(g_mu);
    if (handle < (int)g_open.size()) hipEventRecord(g_open[(size_t)handle].e1, s);
}

}  // namespace gx

using namespace gx;

extern "C" {

int gefenx_profile_enable(int on) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_enabled = on != 0;
    return GEFENX_OK;
}

int gefenx_profile_reset(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& r : g_open) {
        hipEventSynchronize(r.e1);
        g_pool.push_back(r.e0);
        g_pool.push_back(r.e1);
    }
    g_open.clear();
    return GEFENX_OK;
}

int gefenx_profile_read(int kind, double* total_ms, int64_t* launches, double* algo_bytes,
                        double* algo_flops) {
    if (kind < 0 || kind >= GEFENX_K_COUNT)
        return set_error(GEFENX_EINVAL, "gefenx_profile_read: bad kernel kind %d", kind);
    std::lock_guard<std::mutex> lk(g_mu);
    double ms = 0.0, bytes = 0.0, flops = 0.0;
    int64_t n = 0;
    for (auto& r : g_open) {
        if (r.kind != kind) continue;
        if (hipEventSynchronize(r.e1) != hipSuccess)
            return set_error(GEFENX_ELAUNCH, "gefenx_profile_read: event synchronisation failed");
        float t = 0.0f;
        if (hipEventElapsedTime(&t, r.e0, r.e1) != hipSuccess)
            return set_error(GEFENX_ELAUNCH, "gefenx_profile_read: elapsed-time query failed");
        ms += (double)t;
        bytes += r.bytes;
        flops += r.flops;
        ++n;
    }
    if (total_ms) *total_ms = ms;
    if (launches) *launches = n;
    if (algo_bytes) *algo_bytes = bytes;
    if (algo_flops) *algo_flops = flops;
    return GEFENX_OK;
}

}  // extern "C"
