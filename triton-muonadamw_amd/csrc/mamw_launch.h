// Kernel launch wrapper with opt-in per-dispatch timing.
//
// When profiling is on (mamw_prof_start), every launch made through
// mamw::launch() is bracketed by a pair of HIP events bound to that dispatch
// (hipExtLaunchKernelGGL), and a record {kernel id, algorithmic flops and
// bytes, events} is kept until mamw_prof_collect() reads the elapsed times.
// When it is off, launch() is a plain hipLaunchKernelGGL.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "muonadamw_amd.h"

namespace mamw {

// Kernel identifiers reported by the profiler (names: mamw_prof_kernel_name).
enum KernelId : int32_t {
    K_ADAMW_MT = 0,
    K_ADAMW_ONE,
    K_MUON_PREP,
    K_MUON_NORM,
    K_MUON_APPLY0,
    K_MUON_SCALE,
    K_NS_GRAM,
    K_NS_POLY,
    K_NS_UPDATE,
    K_NS_APPLY,
    K_TRANSPOSE,
    K_ADAMW_BIAS,
    K_COUNT
};

// Returns true and two events when profiling is on (and not suspended on
// this thread).
bool prof_take(hipEvent_t* start, hipEvent_t* stop);

// While one of these lives, launches on this thread take no profiler events
// (an entry point that must not allocate creates none).
struct ProfSuspend {
    ProfSuspend();
    ~ProfSuspend();
    ProfSuspend(const ProfSuspend&) = delete;
    ProfSuspend& operator=(const ProfSuspend&) = delete;
};
void prof_push(int32_t kernel, int32_t variant, double flops, double bytes, hipEvent_t start, hipEvent_t stop);

template <typename Kernel, typename... Args>
hipError_t launch(int32_t kernel_id, int32_t variant, double flops, double bytes, Kernel kernel, dim3 grid,
                  dim3 block, hipStream_t stream, Args... args) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (prof_take(&e0, &e1)) {
        hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, e0, e1, 0, args...);
        hipError_t err = hipGetLastError();
        if (err == hipSuccess) prof_push(kernel_id, variant, flops, bytes, e0, e1);
        return err;
    }
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
    return hipGetLastError();
}

}  // namespace mamw
