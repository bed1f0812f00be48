// cascade.hip -- the prefix kernel of the shared-prefix (cascade) path: one workgroup per
// (prefix chunk or tree item, query group, kv head), the body in prefix_body.h.
#include "timeline.h"

PD_TIMELINE_TABLE(prefix)

#include "prefix_body.h"

namespace pdattn {
namespace {

// Two workgroups per CU (two waves per SIMD): one wave's softmax runs while the other's MFMAs
// occupy the matrix core.
__global__ __launch_bounds__(kPrefixThreads, 2) void cascade_prefix_kernel(PrefixArgs a) {
    __shared__ PSmem sm;
    prefix_workgroup(a, sm, blockIdx.x, blockIdx.y, blockIdx.z);
}

}  // namespace

int prefix_rows_per_workgroup() { return kPrefixRows; }

hipError_t launch_cascade_prefix(const PrefixArgs& a, int G, int qtiles, hipStream_t s) {
    (void)G;
    if (a.Hkv <= 0) return hipSuccess;
    if (a.items) {
        // num_chunks = number of items
        if (a.num_chunks <= 0) return hipSuccess;
        cascade_prefix_kernel<<<dim3(a.num_chunks, 1, a.Hkv), kPrefixThreads, 0, s>>>(a);
        return hipGetLastError();
    }
    if (a.num_chunks <= 0 || qtiles <= 0) return hipSuccess;
    dim3 grid(a.num_chunks, qtiles, a.Hkv);
    cascade_prefix_kernel<<<grid, kPrefixThreads, 0, s>>>(a);
    return hipGetLastError();
}

int occupancy_cascade_prefix(int G) {
    (void)G;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&cascade_prefix_kernel), kPrefixThreads, 0) != hipSuccess)
        return 1;
    return n > 0 ? n : 1;
}

}  // namespace pdattn
