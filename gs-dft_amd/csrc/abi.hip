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
unsigned long long* g_work_dev = nullptr;   // kProfCount work counters on g_work_device
int g_work_device = -1;
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

int read_back(void* host, const void* dev, size_t bytes, hipStream_t s, const char* what) {
    const hipError_t ec = hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, s);
    const hipError_t es = hipStreamSynchronize(s);
    if (ec != hipSuccess) return hip_fail(ec, what);
    if (es != hipSuccess) return hip_fail(es, what);
    return GSDFT_OK;
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

unsigned long long* profile_work_counter(int id) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (!g_prof_on || !g_work_dev || id < 0 || id >= kProfCount) return nullptr;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev != g_work_device) return nullptr;
    return g_work_dev + id;
}

}  // namespace gsdft

using namespace gsdft;

extern "C" int gsdft_abi_version(void) { return 1; }

extern "C" const char* gsdft_last_error(void) { return g_err; }

extern "C" int gsdft_profile_enable(int on) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof_on = on != 0;
    if (g_prof_on && !g_work_dev) {
        GSDFT_HIP(hipGetDevice(&g_work_device));
        GSDFT_HIP(hipMalloc((void**)&g_work_dev, sizeof(unsigned long long) * kProfCount));
        GSDFT_HIP(hipMemset(g_work_dev, 0, sizeof(unsigned long long) * kProfCount));
    }
    return GSDFT_OK;
}

extern "C" int gsdft_profile_read_work(int id, uint64_t* units, int reset) {
    if (id < 0 || id >= kProfCount || !units)
        return fail(GSDFT_ERR_ARG, "gsdft_profile_read_work: bad id");
    std::lock_guard<std::mutex> lk(g_prof_mu);
    *units = 0;
    if (!g_work_dev) return GSDFT_OK;
    int dev = -1;
    GSDFT_HIP(hipGetDevice(&dev));
    GSDFT_HIP(hipSetDevice(g_work_device));
    unsigned long long v = 0;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(&v, g_work_dev + id, sizeof v, hipMemcpyDeviceToHost);
    if (e == hipSuccess && reset) e = hipMemset(g_work_dev + id, 0, sizeof v);
    (void)hipSetDevice(dev);
    if (e != hipSuccess) return hip_fail(e, "gsdft_profile_read_work");
    *units = (uint64_t)v;
    return GSDFT_OK;
}

extern "C" int gsdft_profile_read(int id, double* total_ms, int64_t* launches, int reset) {
    if (id < 0 || id >= kProfCount || !total_ms || !launches)
        return fail(GSDFT_ERR_ARG, "gsdft_profile_read: bad id");
    std::lock_guard<std::mutex> lk(g_prof_mu);
    // Every recorded pair is read and destroyed, and the list is emptied, on every path: a pair
    // left behind after an error would be read again after its events were destroyed.
    hipError_t first = hipSuccess;
    for (auto& ev : g_open[id]) {
        hipError_t e = hipEventSynchronize(ev.stop);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.start, ev.stop);
        if (e == hipSuccess) {
            g_total_ms[id] += ms;
            g_launches[id] += 1;
        } else if (first == hipSuccess) {
            first = e;
        }
        (void)hipEventDestroy(ev.start);
        (void)hipEventDestroy(ev.stop);
    }
    g_open[id].clear();
    if (first != hipSuccess) return hip_fail(first, "gsdft_profile_read");
    *total_ms = g_total_ms[id];
    *launches = g_launches[id];
    if (reset) {
        g_total_ms[id] = 0.0;
        g_launches[id] = 0;
    }
    return GSDFT_OK;
}
