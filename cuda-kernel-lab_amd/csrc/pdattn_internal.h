// pdattn_internal.h -- declarations shared by the host planner (api.cpp) and the HIP kernel
// translation units. Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/pdattn.h"

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
    // Non-null (one chunk per sequence, nothing else to merge): the final fp16 out and lse are
    // written here instead of the partial slots; a merge of one partial state would copy it.
    _Float16*       out;
    float*          lse;
    int B, Hq, Hkv, num_chunks, chunk_tokens, kv_start, chunk_base, part_stride;
    float scale_log2;         // sm_scale * log2(e)
};

// Balanced decode: the host planner gives each workgroup a range of pages of one kv head -- by
// default range g of the page sequence cut into W / Hkv equal ranges for workgroup g * Hkv + h,
// kv head h; or the units [U w / W, U (w+1) / W) of the pairs' chunks, kv head fastest -- cut into
// segments (one per sequence or chunk piece), described in desc[w * kBalDescInts ..]:
//   desc[0] = number of segments; desc[1] = the plan's tag (a launch whose tag argument differs
//   finds someone else's bytes there and does nothing); segment s at desc[8 + kSegInts * s] =
//   {b, kvh, qa, npg, t0, t1, jpos, slot}: sequence b, kv head kvh, pages [qa, qa + npg) of the
//   workgroup's page list, tokens [t0, t1) of the sequence (t0 = first token of its first page),
//   page-table position jpos of its first page (relative to kv_indptr[0]), and the partial slot
//   it writes (-1: the segment is the whole pair and writes the final out / lse).
constexpr int kSegMax = 24;                // segments per workgroup
constexpr int kStepSegMax = 8;             // segments per workgroup of the fused cascade step at G = 8
constexpr int kSegInts = 8;
constexpr int kBalDescInts = 8 + kSegMax * kSegInts;
constexpr int kRangeMax = 2048;            // pages per workgroup (page ids staged in LDS)

struct BalArgs {
    const _Float16* q;
    const uint8_t*  k;
    const uint8_t*  v;
    const int32_t*  kv_indices;   // offset by kv_indptr[0]
    _Float16*       out;
    float*          lse;
    const int32_t*  desc;         // [W * kBalDescInts]
    float*          part_o;       // [slots * G * 128] partial outputs (normalized)
    float*          part_lse;     // [slots * G]
    int B, Hq, Hkv, W;
    float scale_log2;             // sm_scale * log2(e)
    // Partial layout: 0 = slot-major (head h of slot s at s * G + h, the planner's slots); > 0 =
    // row-major with this stride (row r = b * Hq + h, slot s at r * part_stride + s: the layout of
    // the reference's decode_partial, where s = chunk_base + chunk)
    int part_stride;
    // > 0: a page-range plan of that many groups; workgroup w = g * Hkv + kvh owns the pages
    // [nnz g / ngroups, nnz (g + 1) / ngroups) of kv_indices (its page list, in order)
    int ngroups;
    int nnz;
    int tag;                      // the plan's tag, expected in desc[1] of every block (host plans)
    // >= 0 (page-range plans of one sequence): every segment of every workgroup is of sequence
    // qrow_b, so a workgroup's q rows (kv head w % Hkv) are loaded with its descriptor block
    int qrow_b = -1;
};

// The reference-shaped uniform split (decode_partial / decode_attention) run by the balanced
// workgroup body: item i = (pair, chunk) with chunk = i % num_chunks, pair = b * Hkv + kvh =
// i / num_chunks covers keys [kv_start + chunk * chunk_tokens, + chunk_tokens) of its sequence.
// Workgroup w of d.W takes the items w, w + W, ... (at most per_wg of them) and builds their
// segment descriptors itself from the device page table, so no host plan is involved. The
// BalArgs come first: the body reads them through the kernel argument pointer.
struct UniArgs {
    BalArgs         d;            // d.kv_indices is not offset; d.out != null: write out / lse
    const int32_t*  kv_indptr;
    const int32_t*  kv_last;
    int kv_start, chunk_tokens, num_chunks, chunk_base, n_items, per_wg;
};

// The drop-in decode_attention with the work cut into equal page ranges on the device, with no
// host plan (pdattn_decode_attention_balanced). Sequence b attends keys [kv_start, kv_start + span)
// of its own (span = num_chunks * chunk_tokens, the reference's clip), i.e. c_b of its pages;
// the attended pages of all sequences, in page-table order, are cut into d.ngroups equal ranges,
// and workgroup g * Hkv + kvh takes range g for kv head kvh: every workgroup loads kv_indptr and
// kv_last_page_len, forms the prefix sums of c_b itself and cuts its range into segments (one per
// sequence piece, at most B <= kDevMaxB sequences). A piece that is a whole sequence writes the
// final out / lse; the pieces of a split sequence write partial slot 2 w (the piece that starts
// the range, the sequence having started before it) or 2 w + 1 (the piece that ends the range,
// the sequence going on after it), slot-major [2 W, G, 128]. A workgroup with an empty range
// marks both its slots empty (lse = -inf). Workgroup 0 writes the prefix sums for the merge.
constexpr int kDevMaxB = 1023;
struct DevArgs {
    BalArgs         d;            // d.kv_indices not offset; d.ngroups ranges; d.part_o / d.part_lse the slots
    const int32_t*  kv_indptr;
    const int32_t*  kv_last;
    int32_t*        prefix;       // [B + 1]: attended pages of the sequences before b
    int64_t         span;         // keys [kv_start, kv_start + span) of each sequence
    int             kv_start;
};

// The merge after it: one workgroup per row (b, q head). A sequence whose pages lie in ranges
// g0 < g1 merges range g0's slot 2 w + 1 and the slots 2 w of ranges g0 + 1 .. g1, in that order.
struct DevMergeArgs {
    const int32_t*  prefix;
    const float*    part_o;
    const float*    part_lse;
    _Float16*       out;
    float*          lse;
    int B, Hq, Hkv, G, ngroups;
};

// Merge of split pairs (and of every pair when extra partials are given). `list` starts with a
// header {tag, n_entries, cmax, 0}; entry e (at list[4 + 4 e]) is {b, kvh, slot0, nc}: the
// nc >= 0 partial slots slot0 .. slot0 + nc - 1 of the pair, in order, then the n_extra extra
// partials of each of its G rows. With cmax > 0 the slots are laid out by entry, slot0 = e * cmax
// (nc <= cmax), so the partials' addresses do not depend on the list and are loaded in the same
// round trip as the entry. With n_extra > 0 the list holds every pair in (b, kvh) order: entry e is
// pair e, so its rows (and their extra partials) are known from e as well.
struct MergeArgs {
    const int32_t*  list;         // [4 + n_entries * 4]
    const float*    part_o;
    const float*    part_lse;
    const float*    extra_o;      // [B*Hq, n_extra, 128] or null
    const float*    extra_lse;    // [B*Hq, n_extra]
    _Float16*       out;
    float*          lse;
    int B, Hq, Hkv, G, n_extra;
    int cmax;                     // > 0: slots laid out by entry (see above)
    int n_slots;                  // partial slots in the workspace (a listed range beyond is refused)
    int tag;                      // expected in the list header (else the launch does nothing)
};

// Paged KV append: token t (of n) of sequence batch_idx[t] at position positions[t].
struct AppendArgs {
    const void*     k_new;        // [n, Hkv, 128] fp16
    const void*     v_new;
    void*           k_cache;      // [num_pages, 16, Hkv, 128] fp16
    void*           v_cache;
    const int32_t*  kv_indptr;
    const int32_t*  kv_indices;
    const int32_t*  batch_idx;
    const int32_t*  positions;
    int32_t*        n_invalid;    // optional: tokens outside their sequence's pages
    int n, B, Hkv;
    int tpb;                      // tokens per workgroup (set by launch_append_kv)
};

// Arguments of the MFMA shared-prefix kernel.
struct PrefixArgs {
    const _Float16* q;
    const uint8_t*  k;
    const uint8_t*  v;
    const int32_t*  prefix_pages;
    const int32_t*  seqs;         // the ns sequences sharing the prefix (null: 0 .. ns-1)
    // Several prefixes in one launch (the nodes of one depth of a prefix tree): workgroup x
    // takes item items[8 x ..] = {page-table position of its node's first page, offset of the
    // node's members in seqs, members, tokens, chunk tokens, first partial column, chunk, query
    // group}; prefix_pages is then the whole page table. Null: one prefix.
    const int32_t*  items;
    float*          part_o;       // rows b*Hq + h, slot row*part_stride + col0 + chunk
    float*          part_lse;
    int B, Hq, Hkv, prefix_len, chunk_tokens, part_stride, num_chunks;
    int ns, col0;
    float scale_log2;
};

// The fused cascade step: n_dec balanced-decode workgroups (the suffix, plan in `d`) followed by
// n_pre prefix workgroups (p.num_chunks items x Hkv kv heads, item table in p.items). The BalArgs
// come first: the decode body reads them through the kernel argument pointer.
struct StepArgs {
    BalArgs    d;
    PrefixArgs p;
    int n_dec, n_pre;
};

// Kernel launchers (defined in the .hip files). Each returns the hipError_t of the launch.
hipError_t launch_decode_partial(const PartialArgs& a, int G, hipStream_t s);
hipError_t launch_merge_states(const float* part_o, const float* part_lse, _Float16* out,
                               float* lse, int rows, int num_chunks, hipStream_t s);
hipError_t launch_decode_balanced(const BalArgs& a, int G, hipStream_t s);
// The paired variant of a page-range plan (two kv heads per workgroup, W / 2 workgroups; G in
// 1, 2, 4 and Hkv even).
hipError_t launch_decode_pair(const BalArgs& a, int G, hipStream_t s);
hipError_t launch_decode_uniform(const UniArgs& a, int G, hipStream_t s);
hipError_t launch_merge_split(const MergeArgs& a, int n_entries, hipStream_t s);
hipError_t launch_decode_ranges(const DevArgs& a, int G, hipStream_t s);
hipError_t launch_merge_ranges(const DevMergeArgs& a, hipStream_t s);
hipError_t launch_fill_i32(int32_t* p, int32_t value, size_t n, hipStream_t s);
hipError_t launch_cascade_prefix(const PrefixArgs& a, int G, hipStream_t s);
hipError_t launch_cascade_step(const StepArgs& a, int G, hipStream_t s);
hipError_t launch_append_kv(const AppendArgs& a, int cus, hipStream_t s);
hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* sink, int grid, hipStream_t s);
hipError_t launch_flush(void* buf, size_t bytes, int grid, hipStream_t s);

// The uniform split behind decode_attention (api.cpp), shared by the no-allocation entry point:
// argument checks (a status; PDATTN_OK for B = 0 too), and the launches with the partial states
// at part_o / part_lse (B * Hq * part_stride slots; unused when num_chunks = 1).
int decode_attention_check(const pdattn_decode_params* p, int G, int variant, const void* out,
                           const float* lse);
int decode_attention_launch(const pdattn_decode_params* p, int G, void* out, float* lse, float* part_o,
                            float* part_lse, hipStream_t s);
// Sets the message pdattn_last_error returns and passes the status through.
int report_error(int status, const char* what);

// Occupancy (workgroups per CU) of the kernels, queried from the runtime.
int occupancy_decode_partial(int G);
int occupancy_decode_balanced(int G);
int occupancy_cascade_prefix(int G);
int occupancy_cascade_step(int G);   // workgroups of the fused step per CU
int prefix_rows_per_workgroup();

}  // namespace pdattn
