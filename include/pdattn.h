/*
 * pdattn.h -- C ABI of the MI355X (gfx950) paged split-KV GQA decode attention library.
 *
 * Drop-in boundary for the decode-attention path of qilem/cuda-kernel-lab
 * (01_decode_attention.cu). That file has no extern "C" layer: its interface is a set of C++
 * free functions and kernels called from its own main(). Each entry point below replaces one of
 * them (cited at the declaration) with the same argument meaning, exposed as plain C so that any
 * FFI (ctypes, cgo, JNI, N-API) can bind it:
 *   - device pointers are passed as `void*` / typed pointers, sizes as ints / size_t;
 *   - a HIP stream is passed as `void*` (a hipStream_t; NULL = the default stream);
 *   - every function returns a pdattn_status (0 = success) instead of calling exit(), which is
 *     what the reference does on any error (common/bench.cuh:21-29, 01:285-286).
 *
 * Tensor layouts (identical to the reference, 01_decode_attention.cu:5-9, 112):
 *   q          [B, Hq, 128]                fp16
 *   k_cache,
 *   v_cache    [num_pages, 16, Hkv, 128]   fp16; element (page, slot, kvh, d) at
 *                                          ((page*16 + slot)*Hkv + kvh)*128 + d
 *   kv_indptr [B+1], kv_indices [nnz], kv_last_page_len [B]   int32 CSR page table (FlashInfer)
 *   out        [B, Hq, 128] fp16;  lse [B, Hq] fp32 (natural log of the scaled scores)
 * q head h reads kv head h / G with G = Hq / Hkv in {1, 2, 4, 8}; head_dim is 128; page size 16.
 * An empty sequence (no pages) yields out = 0, lse = -inf. kv_indices is read only at the
 * positions [kv_indptr[b], kv_indptr[b+1]) of the sequences' pages: when every sequence is empty
 * it may point at a buffer of no elements (but not be NULL).
 */
#ifndef PDATTN_H
#define PDATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PDATTN_HEAD_DIM 128
#define PDATTN_PAGE_SIZE 16
#define PDATTN_SCHEDULE_SEGMENTS 24    /* segments per workgroup in a plan's schedule     */
#define PDATTN_SCHEDULE_WG_INTS 200    /* int32 per workgroup in a plan's schedule        */

typedef enum pdattn_status {
    PDATTN_OK = 0,
    PDATTN_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative size, inconsistent chunking      */
    PDATTN_ERR_UNSUPPORTED = 2,      /* G not in {1,2,4,8}, Hq % Hkv != 0                        */
    PDATTN_ERR_PAGE_TABLE = 3,       /* indptr not monotone, last_page_len outside [1,16], page
                                        id outside the cache (pdattn_check_page_table)            */
    PDATTN_ERR_WORKSPACE = 4,        /* caller-provided workspace smaller than required          */
    PDATTN_ERR_HIP = 5,              /* a HIP runtime call failed (detail in pdattn_last_error)  */
    PDATTN_ERR_NOT_READY = 6         /* plan's schedule not (or no longer) in this workspace     */
} pdattn_status;

/* Name of a status code. */
const char* pdattn_strerror(int status);
/* Detail message of the last failing call on this host thread ("" if none). */
const char* pdattn_last_error(void);

/* Launch argument block. Same fields, order and meaning as DecodeParams
 * (01_decode_attention.cu:51-65). part_o is [B*Hq, part_stride, 128] fp32 holding normalized
 * partial outputs; part_lse is [B*Hq, part_stride]. Chunk c of a sequence covers keys
 * [kv_start + c*chunk_tokens, min(seq_len, kv_start + (c+1)*chunk_tokens)) and writes slot
 * chunk_base + c. */
typedef struct pdattn_decode_params {
    const void*    q;
    const void*    k_cache;
    const void*    v_cache;
    const int32_t* kv_indptr;
    const int32_t* kv_indices;
    const int32_t* kv_last_page_len;
    float*         part_o;
    float*         part_lse;
    int32_t B, Hq, Hkv, num_chunks, chunk_tokens;
    int32_t kv_start;
    int32_t chunk_base;
    int32_t part_stride;
    float   sm_scale;
} pdattn_decode_params;

/* Device workspace. Replaces Workspace (01_decode_attention.cu:314). The reference grows its
 * workspace inside decode_attention with cudaFree/cudaMalloc; here a workspace that the library
 * allocated (owned = 1, or base == NULL) is grown the same way, while caller-provided memory
 * (owned = 0) is never replaced: a call that needs more returns PDATTN_ERR_WORKSPACE. Reserve
 * the required size up front (pdattn_workspace_reserve) to keep every call allocation-free. */
typedef struct pdattn_workspace {
    void*  base;
    size_t bytes;
    int    owned;
} pdattn_workspace;

/* Grow `ws` to at least `bytes` with hipMalloc (ensure_workspace, 01_decode_attention.cu:648-654).
 * Synchronizes the device before freeing an old owned buffer. */
int pdattn_workspace_reserve(pdattn_workspace* ws, size_t bytes);
/* Free an owned workspace and zero the struct (the reference's cudaFree at 01:893). */
void pdattn_workspace_release(pdattn_workspace* ws);

/* Host-side check of a page table against a cache of num_pages pages: kv_indptr [B+1] starts at
 * 0 or more and never decreases, every kv_indices entry in [kv_indptr[0], kv_indptr[B]) lies in
 * [0, num_pages), and every non-empty sequence's kv_last_page_len lies in [1, 16]. Returns
 * PDATTN_OK, PDATTN_ERR_PAGE_TABLE (the first offending position is in pdattn_last_error) or
 * PDATTN_ERR_INVALID_ARGUMENT. The decode kernels read page ids as given, with no bounds check on
 * the device (the launch API carries no cache size): a caller that does not build the table
 * itself checks it here first. No counterpart in the reference, which validates no input. */
int pdattn_check_page_table(const int32_t* h_kv_indptr, const int32_t* h_kv_indices,
                            const int32_t* h_kv_last_page_len, int B, int64_t num_pages);

/* ---- reference-shaped split-KV path (uniform chunks) ------------------------------------- */

/* Chunk count for the uniform split (plan_chunks, 01_decode_attention.cu:289-312): about one
 * workgroup per CU over all (sequence, kv head) pairs (CU count / (B*Hkv), rounded down; the
 * reference uses SM count x occupancy), chunks of at least 256 tokens, chunk_tokens a multiple of
 * 16; force_chunks > 0 overrides. `variant` is accepted for signature parity and must be 0..3. */
int pdattn_plan_chunks(int G, int variant, int B, int Hkv, int max_len, int force_chunks,
                       int* num_chunks, int* chunk_tokens);

/* Partial (o, lse) per chunk into p->part_o / p->part_lse, slot chunk_base + chunk of each row
 * at stride part_stride (decode_partial<G,V>, 01_decode_attention.cu:76-236, launched at
 * 01:327-329). The (chunk, sequence, kv head) items run several per workgroup, about one workgroup
 * per CU; chunks longer than 32752 tokens run one per workgroup. Reads only the device page table. */
int pdattn_decode_partial(const pdattn_decode_params* p, int G, int variant, void* stream);

/* Log-sum-exp merge of `num_chunks` partial states for each of `rows` rows into fp16 out and
 * fp32 lse; rows with every lse = -inf give 0 / -inf (merge_states, 01_decode_attention.cu:238-255). */
int pdattn_merge_states(const float* part_o, const float* part_lse, void* out, float* lse_out,
                        int rows, int num_chunks, void* stream);

/* Bytes of workspace decode_attention needs for B*Hq rows of part_stride partial slots. */
size_t pdattn_decode_workspace_size(int B, int Hq, int part_stride);

/* Where decode_attention places part_o / part_lse inside a workspace (for reading per-chunk lse). */
int pdattn_workspace_partials(const pdattn_workspace* ws, int B, int Hq, int part_stride,
                              float** part_o, float** part_lse);

/* Partial launch then merge launch on `stream`, partials in `ws`; p->part_o / p->part_lse are
 * ignored and taken from the workspace (decode_attention, 01_decode_attention.cu:316-331). */
int pdattn_decode_attention(const pdattn_decode_params* p, int G, int variant, void* out,
                            float* lse, pdattn_workspace* ws, void* stream);

/* Bytes of the device array pdattn_decode_attention_noalloc keeps its partial states in (16 MiB
 * on every GPU the library runs on, held until the process ends). */
#define PDATTN_NOALLOC_SCRATCH_BYTES (16u << 20)

/* pdattn_decode_attention without allocating: the partial states go to the library's own device
 * array (PDATTN_NOALLOC_SCRATCH_BYTES per GPU) instead of a workspace, so the call makes no
 * hipMalloc / hipFree and needs no workspace argument. No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc). The partial states must fit the array: pdattn_decode_workspace_size(B, Hq,
 * part_stride) <= PDATTN_NOALLOC_SCRATCH_BYTES when num_chunks > 1 (one chunk needs none), else
 * PDATTN_ERR_WORKSPACE. Every call on one GPU uses the same array: calls that overlap in time on
 * one GPU (two streams, two host threads) race, and the caller serializes them. */
int pdattn_decode_attention_noalloc(const pdattn_decode_params* p, int G, int variant, void* out,
                                    float* lse, void* stream);

/* decode_attention with the reference-shaped arguments and no host plan, balanced on the device:
 * the pages that each sequence attends (keys [kv_start, kv_start + num_chunks * chunk_tokens),
 * the keys the reference's chunks cover, clipped to the sequence), taken in page-table order over
 * all sequences, are cut into equal ranges, one workgroup per CU and kv head, and every workgroup
 * finds its range from the device kv_indptr / kv_last_page_len itself (prefix sums of the page
 * counts). Sequences of very different lengths are then balanced as by the plan path, where the
 * uniform chunks of pdattn_decode_attention (sized by the longest sequence) leave workgroups
 * idle. A sequence inside one range is written by its workgroup; the pieces of one cut by range
 * boundaries are merged by a second launch, in page order (bitwise deterministic). chunk_base,
 * part_stride, part_o and part_lse of `p` are not used: the partial states live in `ws`, grown
 * like decode_attention's when library-owned (pdattn_decode_balanced_workspace_size bytes). More
 * than 1023 sequences run as pdattn_decode_attention. No counterpart in the reference: it is the
 * uneven chunking the reference names as its next step (README.md:54), behind decode_attention's
 * arguments (01_decode_attention.cu:316-331). */
int pdattn_decode_attention_balanced(const pdattn_decode_params* p, int G, int variant, void* out,
                                     float* lse, pdattn_workspace* ws, void* stream);
/* Workspace bytes pdattn_decode_attention_balanced needs for `p` (0 on an invalid `p`). */
size_t pdattn_decode_balanced_workspace_size(const pdattn_decode_params* p, int G);

/* ---- balanced path (plan / run) ---------------------------------------------------------- */
/* The MI355X path for decode_attention. The planner works on the host, from the host copy of the
 * page table, the way FlashInfer's plan() does. It cuts the pages of all sequences, taken in
 * page-table order, into W / Hkv equal ranges, and gives workgroup g * Hkv + h of a single launch
 * (W = one per CU) range g for kv head h: every workgroup streams the same number of pages, and
 * the Hkv workgroups of a range read the same pages at the same time, each its own 256-byte column
 * of every 2 KB token row, so each token row is read whole while it is open in DRAM. A range that
 * holds pieces of several sequences gives its workgroups one segment per piece.
 *
 * A (sequence, kv head) pair that lies in one workgroup's range is written as the final out / lse
 * by that workgroup. The pieces of a pair split over several workgroups are written as normalized
 * partials and merged by a second, small launch, in a fixed order. The result is bitwise
 * deterministic for a given plan. */
typedef struct pdattn_plan pdattn_plan;

typedef struct pdattn_plan_info {
    int     workgroups;        /* grid size W of the decode launch                        */
    int     pairs;             /* B * Hkv                                                 */
    int     split_pairs;       /* pairs covered by more than one segment                  */
    int     max_contributors;  /* most segments contributing to one pair                  */
    int64_t units;             /* Hkv * nnz page units                                    */
    size_t  workspace_bytes;
    int     chunk_pages;       /* pages per chunk, or per range of the default partition */
    int     segments;          /* segments over all workgroups                            */
    int     merge_entries;     /* pairs merged by the second launch (0: single launch)    */
    int     schedule_ints;     /* int32 count of pdattn_plan_get_schedule's output        */
    int     paired;            /* 1: the decode launch runs workgroups w and w + 1 (kv heads
                                  2k, 2k + 1 of one page range) as one workgroup of the paired
                                  kernel, W / 2 workgroups                                 */
} pdattn_plan_info;

/* Build a plan from host copies of kv_indptr [B+1] and kv_last_page_len [B]. force_workgroups > 0
 * overrides the grid size (one workgroup per CU by default, two at G = 8; it grows when a
 * workgroup would exceed its segment or page limits). At G <= 4 with an even Hkv the default is
 * first planned with two workgroups per CU for the paired kernel, which runs workgroups w and
 * w + 1 (kv heads 2k, 2k + 1 of one page range) as one, its pages staged in LDS; if that plan
 * splits any sequence over workgroups, one workgroup per CU is planned instead (info.paired).
 * chunk_pages > 0, or a grid that is not a
 * multiple of Hkv, selects the other partition: chunks of up to chunk_pages pages (64 by default)
 * of one (sequence, kv head) pair, ordered sequence-major, then by chunk position, kv head
 * fastest, with workgroup w taking the page units [U w / W, U (w+1) / W) of that order (U = Hkv *
 * nnz; the grid is then clamped to U). info.chunk_pages reports the chunk size, or the pages per
 * range of the default partition. */
int pdattn_plan_create(const int32_t* h_kv_indptr, const int32_t* h_kv_last_page_len, int B,
                       int Hq, int Hkv, int force_workgroups, int chunk_pages, pdattn_plan** plan);
int pdattn_plan_get_info(const pdattn_plan* plan, pdattn_plan_info* info);
size_t pdattn_plan_workspace_size(const pdattn_plan* plan);
/* Copy of the plan's schedule (info.schedule_ints int32): per workgroup, the segment count, the
 * plan's tag, 6 unused ints, then up to 24 segments of 8 ints {b, kvh, offset in the workgroup's
 * page list, pages, first token, end token, page-table position of the first page (relative to
 * kv_indptr[0]), partial slot or -1}, 200 ints per workgroup; then the merge list: a header
 * {tag, entries, cmax, 0} and 4 ints per entry {b, kvh, first slot, slots}. With cmax > 0 the
 * partial slots are laid out by entry (entry e's first slot is e * cmax), so that the merge
 * launch loads the entry and the partials in one round trip. The kernels leave a descriptor
 * block or merge list alone whose tag is not the plan's.
 * For inspection and tests; `count` must be at least info.schedule_ints. */
int pdattn_plan_get_schedule(const pdattn_plan* plan, int32_t* out, size_t count);
/* Stream-ordered copy of the plan's schedule into `workspace`. Must precede pdattn_plan_run with
 * that workspace; the plan may then be run any number of times, until another library call writes
 * over the schedule's bytes (another plan's upload or run, or decode_attention's partials in the
 * same memory): pdattn_plan_run then returns PDATTN_ERR_NOT_READY instead of running on what it
 * finds there, and the plan is uploaded again. Writes the library does not make (the caller's own
 * kernels or copies into the workspace, or its memory freed and allocated again at the same
 * address) are not seen by those records: after them the caller uploads again. A run over such
 * bytes computes nothing and writes nothing, since every descriptor block and the merge list
 * carry the plan's tag, which the kernels check (a run therefore needs its upload, not only a
 * workspace of the right size). */
int pdattn_plan_upload(pdattn_plan* plan, void* workspace, size_t bytes, void* stream);
/* Attention for every (sequence, q head) of the planned batch: the decode launch and, when the
 * plan has split pairs or empty sequences, the merge launch. The device page table must hold the
 * same kv_indptr / kv_last_page_len values as the host copy the plan was built from (page ids in
 * kv_indices may change between runs). */
int pdattn_plan_run(const pdattn_plan* plan, const void* q, const void* k_cache,
                    const void* v_cache, const int32_t* kv_indptr, const int32_t* kv_indices,
                    const int32_t* kv_last_page_len, float sm_scale, void* out, float* lse,
                    void* workspace, size_t bytes, void* stream);
/* Measurement hook (no counterpart in the reference, whose harness times whole calls): the same
 * run, making only some of its launches -- PDATTN_RUN_DECODE the decode launch (split pairs leave
 * their partials in the workspace, out / lse of split pairs are not written), PDATTN_RUN_MERGE
 * the merge launch over the partials already in the workspace, PDATTN_RUN_ALL both, which is
 * pdattn_plan_run. For timing each kernel of a step on its own (bench.py); a result is complete
 * only after both parts have run, in that order. */
enum { PDATTN_RUN_DECODE = 1, PDATTN_RUN_MERGE = 2, PDATTN_RUN_ALL = 3 };
int pdattn_plan_run_part(const pdattn_plan* plan, const void* q, const void* k_cache,
                         const void* v_cache, const int32_t* kv_indptr, const int32_t* kv_indices,
                         const int32_t* kv_last_page_len, float sm_scale, void* out, float* lse,
                         void* workspace, size_t bytes, void* stream, int parts);
void pdattn_plan_destroy(pdattn_plan* plan);

/* ---- shared-prefix (cascade) path --------------------------------------------------------- */

/* Longest run of physical pages that every sequence starts with, keeping at least one private
 * page per sequence; 0 when B < 2 (shared_prefix_pages, 01_decode_attention.cu:634-646).
 * Host arrays. Returns the page count (>= 0) or a negative pdattn_status. */
int pdattn_shared_prefix_pages(const int32_t* h_indptr, const int32_t* h_indices, int B);

/* Argument block of the prefix kernel. Same fields and meaning as PrefixParams
 * (01_decode_attention.cu:473-482): prefix_pages are the physical pages of the shared prefix in
 * order; the kernel writes partial slot `chunk` of every (sequence, q head) row it covers. */
typedef struct pdattn_prefix_params {
    const void*    q;
    const void*    k_cache;
    const void*    v_cache;
    const int32_t* prefix_pages;
    float*         part_o;
    float*         part_lse;
    int32_t B, Hq, Hkv, prefix_len, chunk_tokens, part_stride;
    float   sm_scale;
} pdattn_prefix_params;

/* Prefix partials on fp16 MFMA, one partial slot per prefix chunk: slot c covers prefix keys
 * [c*chunk_tokens, min(prefix_len, (c+1)*chunk_tokens)) (cascade_prefix,
 * 01_decode_attention.cu:484-632; chunk count = ceil(prefix_len / chunk_tokens)). */
int pdattn_cascade_prefix(const pdattn_prefix_params* p, void* stream);

typedef struct pdattn_cascade_plan pdattn_cascade_plan;

/* How pdattn_cascade_decode runs the prefix pass and the suffix decode (pdattn_cascade_set_mode).
 * FUSED: one launch whose first workgroups decode the suffix and whose others run the prefix
 * items; both roles are 4-wave workgroups small enough for a CU to hold one of each, so every CU
 * streams suffix pages while its matrix core works on the prefix; the default (at G = 8 the
 * decode role uses a compact LDS layout so that it fits). SERIAL: the prefix launch, then the
 * suffix decode (the reference's order, cascade_decode 01_decode_attention.cu:703-712). TWO_STREAMS:
 * the prefix launch forked onto a second stream owned by the plan, joined before the merge. All
 * three compute the same partials with the same kernels' arithmetic: the results are bitwise
 * equal. The merge launch follows in every mode. */
#define PDATTN_CASCADE_FUSED       0
#define PDATTN_CASCADE_SERIAL      1
#define PDATTN_CASCADE_TWO_STREAMS 2

typedef struct pdattn_cascade_info {
    int    use;             /* 1 when a shared prefix of >= min_prefix tokens was found  */
    int    prefix_tokens;   /* Lp (of the first node)                                   */
    int    prefix_chunks;   /* prefix partial slots per row                            */
    int    prefix_workgroups;
    int    suffix_workgroups;
    size_t workspace_bytes;
    int    nodes;           /* shared-prefix nodes (1 for the reference's rule)        */
    int    levels;          /* depth of the node tree                                  */
    int    mode;            /* PDATTN_CASCADE_*                                        */
} pdattn_cascade_info;

/* Build the cascade plan (plan_cascade, 01_decode_attention.cu:664-701) from the launch block
 * `base` (its q / caches / device page table / B / Hq / Hkv / sm_scale are used), host copies of
 * indptr, indices and sequence lengths, the device kv_indices pointer, and min_prefix tokens
 * (the reference's default is 256). When no prefix of at least min_prefix tokens is shared,
 * info.use = 0 and pdattn_cascade_decode runs the plain balanced decode. */
int pdattn_cascade_plan_create(const pdattn_decode_params* base, const int32_t* h_indptr,
                               const int32_t* h_indices, const int32_t* h_lens,
                               const int32_t* d_indices, int min_prefix,
                               pdattn_cascade_plan** plan);
/* Multi-level cascade: the same decode for a batch whose sequences share prefixes in a tree (a
 * prefix shared by all, then longer ones shared by subgroups, ...). No counterpart in the
 * reference, which lists it as not done (README.md:73). The planner walks the host page table:
 * a group of sequences that hold the same page at some position extends a node while every
 * member holds the same page and keeps a page of its own after it; a node of at least
 * min_prefix tokens is decoded once for all its members on fp16 MFMA, and the group splits by
 * the page that follows. Each sequence's remaining pages go through the balanced decode, and
 * every row merges its suffix partial with the partials of all its nodes, in a fixed order. */
int pdattn_cascade_tree_plan_create(const pdattn_decode_params* base, const int32_t* h_indptr,
                                    const int32_t* h_indices, const int32_t* h_lens,
                                    const int32_t* d_indices, int min_prefix,
                                    pdattn_cascade_plan** plan);
int pdattn_cascade_plan_get_info(const pdattn_cascade_plan* plan, pdattn_cascade_info* info);
/* Prefix pass, suffix decode and merge on `stream` (cascade_decode, 01_decode_attention.cu:703-712),
 * as the plan's mode says. The first call with a given workspace uploads the plan's schedule into
 * it (stream-ordered), and so does any later call after another library call (another plan's
 * decode, decode_attention) has written over it: plans may share one pdattn_workspace. */
int pdattn_cascade_decode(pdattn_cascade_plan* plan, void* out, float* lse, pdattn_workspace* ws,
                          void* stream);
/* Choose how the prefix pass and the suffix decode run (PDATTN_CASCADE_*): both overlap (FUSED,
 * TWO_STREAMS) or not (SERIAL). The reference lists prefix/suffix overlap as not done
 * (README.md:73). FUSED is rejected (PDATTN_ERR_UNSUPPORTED) where its workgroups do not fit two
 * per CU. The TWO_STREAMS stream is created on first use with the default priority; the step
 * stays graph-capturable in every mode. */
int pdattn_cascade_set_mode(pdattn_cascade_plan* plan, int mode);
void pdattn_cascade_plan_destroy(pdattn_cascade_plan* plan);

/* ---- paged KV append ---------------------------------------------------------------------- */

/* Write n new tokens' K and V rows ([n, Hkv, 128] fp16 each) into the paged caches. The page
 * table already describes the caches after the append (the caller has allocated the pages and
 * set kv_indptr / kv_last_page_len, as with FlashInfer's append_paged_kv_cache): token t, at
 * position positions[t] of sequence batch_idx[t], goes to page kv_indices[kv_indptr[b] +
 * pos / 16], slot pos % 16, for every kv head. Layout as in the decode path
 * (01_decode_attention.cu:5-9, 112). A token whose sequence or position is out of range is
 * skipped and counted in *n_invalid (device int32, optional; the caller zeroes it). No
 * counterpart in the reference, which builds its caches on the host (01:402-431); this is the
 * write side of the same page format. */
int pdattn_append_kv(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                     const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* batch_idx,
                     const int32_t* positions, int n, int B, int Hkv, int32_t* n_invalid,
                     void* stream);

/* ---- measurement helpers ------------------------------------------------------------------ */

/* Streams `bytes` (a multiple of 16) with 16-byte loads and folds them into one word, written
 * to *sink only on a sentinel match (stream_read, 01_decode_attention.cu:257-265). */
int pdattn_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream);

/* Reads `bytes` (a multiple of 16) of `buf` once so that the caches hold none of the data timed
 * next; size it above the 256 MB Infinity Cache. Read-only, so it leaves no dirty lines whose
 * write-back the timed kernel would pay for. Replaces the reference's cudaMemsetAsync flush
 * (common/bench.cuh:120, 159). */
int pdattn_flush_cache(void* buf, size_t bytes, void* stream);

typedef struct pdattn_device_info {
    int  compute_units;
    int  decode_wg_per_cu;     /* occupancy of the decode kernels (G = 4)  */
    int  prefix_wg_per_cu;     /* occupancy of the MFMA prefix kernel      */
    char arch[64];
} pdattn_device_info;
int pdattn_get_device_info(pdattn_device_info* info);

#ifdef __cplusplus
}
#endif
#endif /* PDATTN_H */
