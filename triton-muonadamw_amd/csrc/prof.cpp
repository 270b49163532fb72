// Opt-in per-dispatch timing of the library's kernels (host only).
#include <hip/hip_runtime_api.h>

#include <mutex>
#include <vector>

#include "mamw_launch.h"

namespace mamw {
namespace {

struct Rec {
    int32_t kernel, variant;
    double flops, bytes;
    hipEvent_t start, stop;
};

std::mutex g_mu;
bool g_on = false;
thread_local int g_suspended = 0;  // ProfSuspend nesting depth on this thread
std::vector<Rec> g_recs;
std::vector<hipEvent_t> g_free;  // events ready for reuse

hipEvent_t take_event() {
    if (!g_free.empty()) {
        hipEvent_t e = g_free.back();
        g_free.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Host allocations here may fail: no C++ exception may cross the C ABI, so a
// record or an event that cannot be kept is dropped (an event is destroyed).
void keep_free(hipEvent_t e) {
    try {
        g_free.push_back(e);
    } catch (...) {
        (void)hipEventDestroy(e);
    }
}

void recycle_records() {
    for (Rec& r : g_recs) {
        keep_free(r.start);
        keep_free(r.stop);
    }
    g_recs.clear();
}

const char* const kNames[K_COUNT] = {
    "adamw_mt_kernel", "adamw_one_kernel", "muon_prep_kernel", "muon_norm_kernel", "muon_apply0_kernel",
    "muon_scale_kernel",
    "ns_gemm_kernel:gram", "ns_gemm_kernel:poly", "ns_gemm_kernel:update", "ns_gemm_kernel:apply",
    "transpose_bf16_kernel", "adamw_bias_kernel",
};

}  // namespace

ProfSuspend::ProfSuspend() { ++g_suspended; }
ProfSuspend::~ProfSuspend() { --g_suspended; }

bool prof_take(hipEvent_t* start, hipEvent_t* stop) {
    if (g_suspended) return false;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_on) return false;
    *start = take_event();
    *stop = take_event();
    if (!*start || !*stop) {
        if (*start) keep_free(*start);
        if (*stop) keep_free(*stop);
        return false;
    }
    return true;
}

void prof_push(int32_t kernel, int32_t variant, double flops, double bytes, hipEvent_t start, hipEvent_t stop) {
    std::lock_guard<std::mutex> lk(g_mu);
    try {
        g_recs.push_back(Rec{kernel, variant, flops, bytes, start, stop});
    } catch (...) {
        keep_free(start);
        keep_free(stop);
    }
}

}  // namespace mamw

using namespace mamw;

extern "C" int mamw_prof_start(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    recycle_records();
    g_on = true;
    return MAMW_OK;
}

extern "C" int mamw_prof_stop(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_on = false;
    return MAMW_OK;
}

extern "C" int mamw_prof_collect(mamw_prof_record* out, int capacity, int* count) {
    if (!count) return MAMW_ERR_NULL;
    if (capacity < 0 || (capacity > 0 && !out)) return MAMW_ERR_NULL;
    std::lock_guard<std::mutex> lk(g_mu);
    const int n = int(g_recs.size());
    *count = n;
    if (capacity < n) return n == 0 ? MAMW_OK : MAMW_ERR_TABLE;
    for (int i = 0; i < n; ++i) {
        const Rec& r = g_recs[i];
        hipError_t e = hipEventSynchronize(r.stop);
        if (e != hipSuccess) return int(e);
        float ms = 0.f;
        e = hipEventElapsedTime(&ms, r.start, r.stop);
        if (e != hipSuccess) return int(e);
        out[i].kernel = r.kernel;
        out[i].variant = r.variant;
        out[i].flops = r.flops;
        out[i].bytes = r.bytes;
        out[i].ms = ms;
    }
    recycle_records();
    return MAMW_OK;
}

extern "C" const char* mamw_prof_kernel_name(int kernel) {
    if (kernel < 0 || kernel >= K_COUNT) return "unknown";
    return kNames[kernel];
}
