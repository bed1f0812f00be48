// noalloc.hip -- pdattn_decode_attention_noalloc: the reference-shaped split-KV decode
// (decode_attention) with its partial states in a device array of the library's own instead of a
// workspace, so that the call allocates no memory (for callers under HIP graph capture or in
// serving loops that may not call hipMalloc).
//
// The array, `scratch`, is a file-scope __device__ array: every GPU the library runs on holds its
// own copy (PDATTN_NOALLOC_SCRATCH_BYTES) from when the code object is loaded until the process
// ends. In host code its name is only a host-side stand-in for the symbol; the device address of
// each GPU's copy comes from hipGetSymbolAddress, called once per device with that device current,
// and only that address is passed to kernels. Nothing in it has to start at zero: every partial
// slot the merge reads is written by the partial launch of the same call. Calls on one GPU share
// the array, so calls that overlap in time on one GPU (two streams, two host threads) race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "pdattn_internal.h"

static __device__ __align__(256) unsigned char scratch[PDATTN_NOALLOC_SCRATCH_BYTES];

namespace pdattn {
namespace {

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;   // device address of `scratch` per device (null: not yet looked up)

// The current device's copy of `scratch`, looked up on the first call on that device.
int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return report_error(PDATTN_ERR_HIP, hipGetErrorString(e));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return report_error(PDATTN_ERR_HIP, "hipGetSymbolAddress(scratch) failed");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return PDATTN_OK;
}

}  // namespace
}  // namespace pdattn

extern "C" int pdattn_decode_attention_noalloc(const pdattn_decode_params* p, int G, int variant,
                                               void* out, float* lse, void* stream) {
    using namespace pdattn;
    if (int st = decode_attention_check(p, G, variant, out, lse)) return st;
    if (p->B == 0) return PDATTN_OK;
    // with one chunk per sequence the partial launch writes out / lse itself: no partial states
    const size_t need = p->num_chunks == 1 ? 0 : pdattn_decode_workspace_size(p->B, p->Hq, p->part_stride);
    if (need > PDATTN_NOALLOC_SCRATCH_BYTES)
        return report_error(PDATTN_ERR_WORKSPACE,
                            "the partial states need more than the PDATTN_NOALLOC_SCRATCH_BYTES the "
                            "no-allocation array holds: fewer chunks, or pdattn_decode_attention");
    void* base = nullptr;
    if (int st = scratch_address(&base)) return st;
    // the layout of pdattn_workspace_partials: part_o, then part_lse at the next 256-byte boundary
    const size_t rows = (size_t)p->B * p->Hq * p->part_stride;
    float* part_o = static_cast<float*>(base);
    float* part_lse = reinterpret_cast<float*>(static_cast<char*>(base) +
                                               (rows * kHeadDim * sizeof(float) + 255) / 256 * 256);
    return decode_attention_launch(p, G, out, lse, part_o, part_lse, static_cast<hipStream_t>(stream));
}
