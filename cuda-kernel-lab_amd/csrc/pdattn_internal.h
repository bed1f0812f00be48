// pdattn_internal.h -- declarations shared by the host planner (api.cpp) and the HIP kernel
// translation units. Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pdattn {

constexpr int kHeadDim = 128;
constexpr int kPage = 16;

// Arguments of the uniform-chunk partial kernel (the reference's decode_partial launch).
struct PartialArgs {
    const _Float16* q;
    const uint8_t*  k;        // byte pointers: addresses are formed in bytes
    const uint8_t*  v;
    const int32_t*  kv_indptr;
    const int32_t*  kv_indices;
    const int32_t*  kv_last;
    float*          part_o;
    float*          part_lse;
    int B, Hq, Hkv, num_chunks, chunk_tokens, kv_start, chunk_base, part_stride;
    float scale_log2;         // sm_scale * log2(e)
};

// Balanced single-launch kernel: per-workgroup descriptor written by the host planner.
// desc[w * kDescInts + 0] = number of segments; segment s at desc[w * kDescInts + 8 + 8 s] =
//   {b, kvh, qa, npg, t0, t1, w1, nc}: sequence b, kv head kvh, pages [qa, qa + npg) of the
//   workgroup's page range, tokens [t0, t1) of the sequence (t0 is the first token of page qa),
//   first contributing workgroup w1 and contributor count nc of the (b, kvh) pair (nc = 1: this
//   workgroup covers the whole pair).
constexpr int kSegMax = 8;                 // segments per workgroup
constexpr int kSegInts = 8;
constexpr int kDescInts = 8 + kSegMax * kSegInts;
constexpr int kRangeMax = 2048;            // pages per workgroup (page ids staged in LDS)

struct StreamKArgs {
    const _Float16* q;
    const uint8_t*  k;
    const uint8_t*  v;
    const int32_t*  kv_indices;
    _Float16*       out;
    float*          lse;
    const int32_t*  desc;         // [W * kDescInts]
    const int32_t*  empty_seq;    // [n_empty] sequences with no pages
    int32_t*        counters;     // [B*Hkv] arrival counters of split pairs (zero between launches)
    float*          part_o;       // [(B*Hkv + W) * G * 128] partial slots, slot = pair + workgroup
    float*          part_lse;     // [(B*Hkv + W) * G]
    // extra partials merged into every row (cascade prefix): [B*Hq, n_extra] slots
    const float*    extra_o;
    const float*    extra_lse;
    int64_t U;                    // Hkv * nnz page units, kv-head-major
    int nnz, jbase;               // pages in the table, kv_indptr[0]
    int B, Hq, Hkv, W, n_empty;
    int n_extra;
    float scale_log2;
};

// Arguments of the MFMA shared-prefix kernel.
struct PrefixArgs {
    const _Float16* q;
    const uint8_t*  k;
    const uint8_t*  v;
    const int32_t*  prefix_pages;
    float*          part_o;       // rows b*Hq + h, slot row*part_stride + chunk
    float*          part_lse;
    int B, Hq, Hkv, prefix_len, chunk_tokens, part_stride, num_chunks;
    float scale_log2;
};

// Kernel launchers (defined in the .hip files). Each returns the hipError_t of the launch.
hipError_t launch_decode_partial(const PartialArgs& a, int G, hipStream_t s);
hipError_t launch_merge_states(const float* part_o, const float* part_lse, _Float16* out,
                               float* lse, int rows, int num_chunks, hipStream_t s);
hipError_t launch_decode_streamk(const StreamKArgs& a, int G, hipStream_t s);
hipError_t launch_fill_i32(int32_t* p, int32_t value, size_t n, hipStream_t s);
hipError_t launch_cascade_prefix(const PrefixArgs& a, int G, int qtiles, hipStream_t s);
hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* sink, int grid, hipStream_t s);
hipError_t launch_flush(void* buf, size_t bytes, int grid, hipStream_t s);

// Occupancy (workgroups per CU) of the kernels, queried from the runtime.
int occupancy_decode_partial(int G);
int occupancy_decode_streamk(int G);
int occupancy_cascade_prefix(int G);
int prefix_rows_per_workgroup();

}  // namespace pdattn
