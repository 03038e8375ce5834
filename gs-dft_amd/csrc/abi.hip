// C ABI glue: error messages, version, and the event-based kernel timer.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

#include "internal.h"

namespace gsdft {

namespace {
thread_local char g_err[1024] = "";

struct EventPair {
    hipEvent_t start, stop;
};

std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<EventPair> g_open[kProfCount];     // recorded, not yet read
std::vector<hipEvent_t> g_pending_start[kProfCount];
double g_total_ms[kProfCount] = {0};
int64_t g_launches[kProfCount] = {0};
}  // namespace

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(GSDFT_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

void profile_begin(int id, hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (!g_prof_on) return;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return;
    (void)hipEventRecord(e, s);
    g_pending_start[id].push_back(e);
}

void profile_end(int id, hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (!g_prof_on || g_pending_start[id].empty()) return;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return;
    (void)hipEventRecord(e, s);
    g_open[id].push_back(EventPair{g_pending_start[id].back(), e});
    g_pending_start[id].pop_back();
}

}  // namespace gsdft

using namespace gsdft;

extern "C" int gsdft_abi_version(void) { return 1; }

extern "C" const char* gsdft_last_error(void) { return g_err; }

extern "C" int gsdft_profile_enable(int on) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof_on = on != 0;
    return GSDFT_OK;
}

extern "C" int gsdft_profile_read(int id, double* total_ms, int64_t* launches, int reset) {
    if (id < 0 || id >= kProfCount || !total_ms || !launches)
        return fail(GSDFT_ERR_ARG, "gsdft_profile_read: bad id");
    std::lock_guard<std::mutex> lk(g_prof_mu);
    for (auto& ev : g_open[id]) {
        GSDFT_HIP(hipEventSynchronize(ev.stop));
        float ms = 0.f;
        GSDFT_HIP(hipEventElapsedTime(&ms, ev.start, ev.stop));
        g_total_ms[id] += ms;
        g_launches[id] += 1;
        (void)hipEventDestroy(ev.start);
        (void)hipEventDestroy(ev.stop);
    }
    g_open[id].clear();
    *total_ms = g_total_ms[id];
    *launches = g_launches[id];
    if (reset) {
        g_total_ms[id] = 0.0;
        g_launches[id] = 0;
    }
    return GSDFT_OK;
}
