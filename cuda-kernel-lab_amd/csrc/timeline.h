// timeline.h -- optional per-workgroup timestamps, compiled in only with -DPDATTN_TIMELINE (the
// `timeline` target of the Makefile builds lib/timeline/libpdattn.so that way; the library
// proper has none of it).
//
// PD_STAMP(slot) stores s_memrealtime (a 100 MHz counter) from thread 0 of the workgroup into
// row = linear workgroup index, column slot, of a device table that each translation unit
// defines once (PD_TIMELINE_TABLE) together with its extern "C" reader and reset. The stamps
// take nothing out of the kernels: they time the phases of the code that runs.
#pragma once

#include <hip/hip_runtime.h>

namespace pdattn {
constexpr int kTimelineRows = 8192;   // workgroups recorded per launch
constexpr int kTimelineSlots = 32;    // stamps per workgroup
}  // namespace pdattn

#ifdef PDATTN_TIMELINE

// (static: one table per translation unit, read through that unit's functions)
#define PD_TIMELINE_TABLE(NAME)                                                                    \
    static __device__ unsigned long long pd_timeline[pdattn::kTimelineRows * pdattn::kTimelineSlots]; \
    extern "C" int pdattn_timeline_read_##NAME(void* dst, size_t bytes) {                          \
        if (bytes > sizeof(pd_timeline)) bytes = sizeof(pd_timeline);                              \
        return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(pd_timeline), bytes, 0,                    \
                                        hipMemcpyDeviceToHost);                                    \
    }                                                                                              \
    extern "C" int pdattn_timeline_reset_##NAME() {                                                \
        void* p = nullptr;                                                                         \
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(pd_timeline));                           \
        if (e == hipSuccess) e = hipMemset(p, 0, sizeof(pd_timeline));                             \
        if (e == hipSuccess) e = hipDeviceSynchronize();                                           \
        return (int)e;                                                                             \
    }

#define PD_STAMP(slot)                                                                             \
    do {                                                                                           \
        const unsigned pd_row = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;    \
        if (threadIdx.x == 0 && pd_row < (unsigned)pdattn::kTimelineRows)                          \
            pd_timeline[(size_t)pd_row * pdattn::kTimelineSlots + (slot)] =                        \
                __builtin_amdgcn_s_memrealtime();                                                  \
    } while (0)

#else

#define PD_TIMELINE_TABLE(NAME)
#define PD_STAMP(slot) do {} while (0)

#endif
