// api.cpp -- C ABI of libpdattn: validation, planning, workspace handling, launch sequencing.
//
// Host side of the decode-attention path of qilem/cuda-kernel-lab (01_decode_attention.cu),
// re-designed for one MI355X: planners size grids from the runtime's occupancy query and the CU
// count, errors are returned as status codes, and workspaces are either caller-provided (never
// reallocated) or library-owned (grown like the reference's Workspace).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/pdattn.h"
#include "pdattn_internal.h"

using namespace pdattn;

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(PDATTN_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define PD_HIP(call)                                              \
    do {                                                          \
        hipError_t e_ = (call);                                   \
        if (e_ != hipSuccess) return hip_fail(e_, #call);         \
    } while (0)

constexpr size_t kAlign = 256;
constexpr int kXcds = 8;   // accelerator complex dies of MI355X, each with its own L2
constexpr int kDefaultChunkPages = 64;
static_assert(PDATTN_SCHEDULE_SEGMENTS == kSegMax && PDATTN_SCHEDULE_WG_INTS == kBalDescInts,
              "schedule layout in pdattn.h matches the kernel's descriptor");
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool valid_group(int G) { return G == 1 || G == 2 || G == 4 || G == 8; }

// Per-device facts cached on first use: CU count, arch name, kernel occupancies.
struct DeviceFacts {
    int cus = 0;
    int occ_partial[9] = {};
    int occ_balanced[9] = {};
    int occ_prefix[9] = {};
    int occ_step[9] = {};
    char arch[64] = {};
};

std::mutex g_dev_mu;
std::vector<DeviceFacts> g_dev;

int device_facts(DeviceFacts* out) {
    int dev = 0;
    PD_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_dev_mu);
    if ((int)g_dev.size() <= dev) g_dev.resize(dev + 1);
    DeviceFacts& f = g_dev[dev];
    if (f.cus == 0) {
        hipDeviceProp_t prop;
        PD_HIP(hipGetDeviceProperties(&prop, dev));
        f.cus = prop.multiProcessorCount;
        snprintf(f.arch, sizeof f.arch, "%s", prop.gcnArchName);
        for (int G : {1, 2, 4, 8}) {
            f.occ_partial[G] = occupancy_decode_partial(G);
            f.occ_balanced[G] = occupancy_decode_balanced(G);
            f.occ_prefix[G] = occupancy_cascade_prefix(G);
            f.occ_step[G] = occupancy_cascade_step(G);
        }
    }
    *out = f;
    return PDATTN_OK;
}

int check_heads(int Hq, int Hkv, int* G) {
    if (Hq <= 0 || Hkv <= 0) return fail(PDATTN_ERR_INVALID_ARGUMENT, "Hq=%d Hkv=%d must be positive", Hq, Hkv);
    if (Hq % Hkv) return fail(PDATTN_ERR_UNSUPPORTED, "Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
    *G = Hq / Hkv;
    if (!valid_group(*G)) return fail(PDATTN_ERR_UNSUPPORTED, "GQA group size %d not in {1,2,4,8}", *G);
    return PDATTN_OK;
}

// Host page table check: indptr monotone from 0..nnz, last_page_len in [1,16] for non-empty.
int check_host_table(const int32_t* indptr, const int32_t* last, int B) {
    if (!indptr || (B > 0 && !last)) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null host page table");
    if (indptr[0] < 0) return fail(PDATTN_ERR_PAGE_TABLE, "kv_indptr[0]=%d is negative", indptr[0]);
    for (int b = 0; b < B; ++b) {
        if (indptr[b + 1] < indptr[b])
            return fail(PDATTN_ERR_PAGE_TABLE, "kv_indptr not monotone at %d (%d > %d)", b, indptr[b], indptr[b + 1]);
        if (indptr[b + 1] > indptr[b] && (last[b] < 1 || last[b] > kPage))
            return fail(PDATTN_ERR_PAGE_TABLE, "kv_last_page_len[%d]=%d outside [1,16]", b, last[b]);
    }
    return PDATTN_OK;
}

int check_decode_params(const pdattn_decode_params* p, int G) {
    if (!p) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null params");
    if (p->B < 0) return fail(PDATTN_ERR_INVALID_ARGUMENT, "B=%d is negative", p->B);
    int g = 0;
    if (int st = check_heads(p->Hq, p->Hkv, &g)) return st;
    if (g != G) return fail(PDATTN_ERR_INVALID_ARGUMENT, "G=%d but Hq/Hkv=%d", G, g);
    if (p->B == 0) return PDATTN_OK;
    if (!p->q || !p->k_cache || !p->v_cache || !p->kv_indptr || !p->kv_indices || !p->kv_last_page_len)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "null device pointer in params");
    if (!aligned16(p->q) || !aligned16(p->k_cache) || !aligned16(p->v_cache))
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "q / k_cache / v_cache must be 16-byte aligned");
    if (p->num_chunks < 1 || p->chunk_tokens < 1)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "num_chunks=%d chunk_tokens=%d must be >= 1", p->num_chunks, p->chunk_tokens);
    if (p->kv_start < 0 || p->chunk_base < 0)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "kv_start / chunk_base must be >= 0");
    if (p->part_stride < p->chunk_base + p->num_chunks)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "part_stride=%d < chunk_base + num_chunks=%d",
                    p->part_stride, p->chunk_base + p->num_chunks);
    if (!std::isfinite(p->sm_scale)) return fail(PDATTN_ERR_INVALID_ARGUMENT, "sm_scale is not finite");
    return PDATTN_OK;
}

PartialArgs to_partial_args(const pdattn_decode_params* p) {
    PartialArgs a;
    a.q = static_cast<const _Float16*>(p->q);
    a.k = static_cast<const uint8_t*>(p->k_cache);
    a.v = static_cast<const uint8_t*>(p->v_cache);
    a.kv_indptr = p->kv_indptr;
    a.kv_indices = p->kv_indices;
    a.kv_last = p->kv_last_page_len;
    a.part_o = p->part_o;
    a.part_lse = p->part_lse;
    a.out = nullptr;
    a.lse = nullptr;
    a.B = p->B;
    a.Hq = p->Hq;
    a.Hkv = p->Hkv;
    a.num_chunks = p->num_chunks;
    a.chunk_tokens = p->chunk_tokens;
    a.kv_start = p->kv_start;
    a.chunk_base = p->chunk_base;
    a.part_stride = p->part_stride;
    a.scale_log2 = p->sm_scale * 1.4426950408889634f;
    return a;
}

// ---- schedules resident in device memory ----------------------------------------------------
// A plan's schedule (segment descriptors and merge list; for a cascade plan also its suffix page
// table, member lists, prefix items and its -inf lse columns) is copied into a workspace once and
// read by every run. Each such copy is recorded here as a byte range owned by the plan's id. Every
// library call that writes device memory (an upload, the partials of a run or of the uniform
// split, the outputs of any launch) drops the records of other owners that its writes overlap,
// and a run first checks that its plan's records are all still there: a schedule that another
// call has overwritten is uploaded again (cascade_decode, which owns its uploads) or reported as
// PDATTN_ERR_NOT_READY (plan_run, whose caller uploads), never run. The records follow host call
// order, which is the device order of calls on one stream. Writes the library does not make (the
// caller's own kernels or copies into a workspace, or freeing it and allocating new memory at the
// same address) are not seen: after those the caller uploads again.
struct Resident {
    uintptr_t lo, hi;
    uint64_t owner;
};
std::mutex g_res_mu;
std::vector<Resident> g_res;
std::atomic<uint64_t> g_next_owner{1};

uint64_t new_owner() { return g_next_owner.fetch_add(1); }

// A plan's schedule tag: a mix of its owner id with the high bit set, so that it is never a small
// integer, a float's usual bit pattern or a fill value such as 0 or -1.
int32_t schedule_tag(uint64_t id) {
    uint64_t x = (id + 0x9E3779B97F4A7C15ull) * 0xBF58476D1CE4E5B9ull;
    x ^= x >> 31;
    const uint32_t t = (uint32_t)(x >> 32) | 0x80000000u;
    return (int32_t)(t == 0xFFFFFFFFu ? 0x8A5A5A5Au : t);
}

void res_drop_locked(uintptr_t lo, uintptr_t hi, uint64_t keep) {
    g_res.erase(std::remove_if(g_res.begin(), g_res.end(),
                               [&](const Resident& r) { return r.owner != keep && r.lo < hi && lo < r.hi; }),
                g_res.end());
}

// The library is about to write [p, p + n): records of owners other than `keep` there are void.
void res_written(const void* p, size_t n, uint64_t keep = 0) {
    if (!p || n == 0) return;
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
    std::lock_guard<std::mutex> lk(g_res_mu);
    res_drop_locked(lo, lo + n, keep);
}

// [p, p + n) now holds part of owner's schedule.
void res_claim(const void* p, size_t n, uint64_t owner) {
    if (!p || n == 0) return;
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
    std::lock_guard<std::mutex> lk(g_res_mu);
    res_drop_locked(lo, lo + n, 0);   // every record there, the owner's own included
    g_res.push_back({lo, lo + n, owner});
}

// Whether [p, p + n) still holds what owner uploaded there.
bool res_holds(const void* p, size_t n, uint64_t owner) {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
    std::lock_guard<std::mutex> lk(g_res_mu);
    for (const Resident& r : g_res)
        if (r.owner == owner && r.lo == lo && r.hi == lo + n) return true;
    return false;
}

void res_forget(uint64_t owner) {
    std::lock_guard<std::mutex> lk(g_res_mu);
    g_res.erase(std::remove_if(g_res.begin(), g_res.end(), [&](const Resident& r) { return r.owner == owner; }),
                g_res.end());
}

// out [rows, 128] fp16 and lse [rows] fp32 of a launch.
void res_written_outputs(const void* out, const void* lse, size_t rows) {
    res_written(out, rows * kHeadDim * sizeof(_Float16));
    res_written(lse, rows * sizeof(float));
}

int ensure_ws(pdattn_workspace* ws, size_t need) {
    if (!ws) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null workspace");
    if (ws->bytes >= need && ws->base) return PDATTN_OK;
    if (ws->base && !ws->owned)
        return fail(PDATTN_ERR_WORKSPACE, "caller-provided workspace holds %zu bytes, %zu needed", ws->bytes, need);
    return pdattn_workspace_reserve(ws, need);
}

}  // namespace

// ---- plans ------------------------------------------------------------------------------------

struct pdattn_plan {
    int B = 0, Hq = 0, Hkv = 0, G = 0;
    int nnz = 0, jbase = 0, W = 1, P = 16;
    int ngroups = 0;                  // > 0: page-range partition of that many groups
    int64_t U = 0;
    int split_pairs = 0, max_contrib = 0, n_entries = 0, n_slots = 0, segments = 0;
    int cmax = 0;                     // > 0: partial slots laid out by merge entry (e * cmax + k)
    bool pair = false;                // page-range plan run by the paired kernel (W / 2 workgroups)
    // workspace layout (bytes from the base)
    size_t off_desc = 0, off_list = 0, off_plse = 0, off_po = 0, ws_bytes = 0;
    std::vector<int32_t> host_blob;   // desc[W * kBalDescInts] followed by the merge list
    void* pinned = nullptr;           // pinned copy of host_blob for stream-ordered upload
    size_t blob_bytes = 0;
    uint64_t id = new_owner();        // owner of its uploaded schedules (resident-schedule records)
    // Written into every descriptor block and the merge list header, and passed to the kernels,
    // which leave a block or list that does not carry it alone (bytes written over since the
    // upload by something the resident-schedule records cannot see).
    int32_t tag = schedule_tag(id);
};

// One node of a shared-prefix tree: the ns sequences seqs[seq_off ..] all hold the same physical
// pages at positions [p0, p1) of their page lists (page-table positions jpos .. of the first
// member), and each keeps at least one page of its own after p1.
struct CascadeNode {
    int p0 = 0, p1 = 0, jpos = 0, depth = 0;
    int seq_off = 0, ns = 0;
    int ctok = 0, nchunks = 0, col0 = 0, qgroups = 0;
};

struct pdattn_cascade_plan {
    int use = 0;
    int Lp = 0;                        // tokens of the first node (the batch-wide prefix, if any)
    int levels = 0;                    // depth of the node tree
    int n_extra = 0;                   // prefix partial columns per row
    std::vector<int> level_items;      // items (workgroups per kv head) of each depth's launch
    int n_items = 0;
    pdattn_decode_params base{};
    const int32_t* d_indices = nullptr;
    std::vector<CascadeNode> nodes;
    pdattn_plan sk;                    // balanced plan of the suffix (or of the whole batch)
    std::vector<int32_t> blob;         // suffix indptr [B+1], suffix indices, node members
    int n_suffix_idx = 0, n_seqs = 0;
    void* pinned = nullptr;
    size_t off_ppo = 0, off_pplse = 0, off_blob = 0, off_sk = 0, ws_bytes = 0;
    uint64_t id = new_owner();         // owner of its blob and -inf columns in a workspace
    // how the prefix and suffix passes run (pdattn_cascade_set_mode); the second stream of the
    // two-stream mode is created on first use
    int mode = PDATTN_CASCADE_SERIAL;
    hipStream_t aux = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
};

namespace {

// Balanced split; see pdattn.h and pdattn_internal.h. Default: page ranges shared by the Hkv
// workgroups of a group (one kv head each), so that the token rows of a page are read whole.
// Otherwise (a forced chunk size, or a grid that is not a multiple of Hkv): chunks of up to P
// pages of one (sequence, kv head) pair, ordered sequence-major, then by chunk position, kv head
// fastest, and workgroup w owns the units [U w / W, U (w+1) / W) of that order. Either walk cuts
// each workgroup's range into one segment per sequence (or chunk) piece. The contributors of a
// pair are its segments in page order; a pair with more than one (or every pair, when `merge_all`
// is set for extra partials) gets consecutive partial slots and an entry in the merge list. W
// grows (doubling) until every workgroup has at most seg_cap (<= kSegMax) segments and kRangeMax
// pages.
int build_balanced_plan(const int32_t* indptr, const int32_t* last, int B, int Hq, int Hkv,
                        int force_wg, int chunk_pages, bool merge_all, pdattn_plan* pl,
                        int seg_cap = 0, bool pairable = false) {
    int G = 0;
    if (int st = check_heads(Hq, Hkv, &G)) return st;
    // at G = 8 the decode kernel stages q rows for at most kStepSegMax segments per workgroup
    const bool wide = G > 4;
    if (seg_cap <= 0) seg_cap = wide ? kStepSegMax : kSegMax;
    if (B < 0) return fail(PDATTN_ERR_INVALID_ARGUMENT, "B=%d is negative", B);
    if (chunk_pages < 0 || chunk_pages > kRangeMax)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "chunk_pages=%d outside [0, %d]", chunk_pages, kRangeMax);
    if (B > 0)
        if (int st = check_host_table(indptr, last, B)) return st;

    pl->B = B;
    pl->Hq = Hq;
    pl->Hkv = Hkv;
    pl->G = G;
    pl->P = chunk_pages > 0 ? chunk_pages : kDefaultChunkPages;
    pl->jbase = B > 0 ? indptr[0] : 0;
    pl->nnz = B > 0 ? indptr[B] - indptr[0] : 0;
    pl->U = (int64_t)Hkv * pl->nnz;

    // grid: one workgroup per CU (the kernel's four waves take one SIMD each; two at G = 8), never more
    // workgroups than page units; a forced size needs no device query
    int64_t W = force_wg;
    // The paired kernel (two kv heads per workgroup, pages staged in LDS) runs a default page-range
    // plan at G <= 4 with an even Hkv: two plan workgroups per CU, one kernel workgroup.
    const bool pair = pairable && force_wg <= 0 && chunk_pages == 0 && !merge_all && !wide &&
                      Hkv % 2 == 0;
    if (W <= 0) {
        DeviceFacts f;
        if (int st = device_facts(&f)) return st;
        // G = 8 (VALU-limited per page): two workgroups per CU, except for the cascade's suffix,
        // whose workgroups share the CUs with the prefix pass
        W = (int64_t)f.cus * (wide && !merge_all ? 2 : 1) * (pair ? 2 : 1);
    }
    // Page-range groups, the default: the pages of all sequences, in page-table order, are cut
    // into NG = W / Hkv equal ranges, and workgroup g * Hkv + h takes range g for kv head h. The
    // Hkv workgroups of a group stream the same pages at the same time, each its own 256-byte
    // column of every 2 KB token row, so each token row of K and V is read whole while it is open
    // in DRAM. A forced chunk size, or a grid that is not a multiple of Hkv, uses the unit ranges
    // below instead (chunks of one kv head, kv head fastest).
    const bool grouped = chunk_pages == 0 && W >= Hkv && W % Hkv == 0;
    if (!grouped) {
        W = std::max<int64_t>(1, std::min<int64_t>(W, std::max<int64_t>(1, pl->U)));
        W = std::max<int64_t>(W, (pl->U + kRangeMax - 1) / kRangeMax);
    }
    if (W > (1 << 28)) return fail(PDATTN_ERR_INVALID_ARGUMENT, "grid too large");

    const int64_t U = pl->U;
    const int P = pl->P;
    const int64_t nnz = pl->nnz;
    const int jbase = pl->jbase;
    auto seq_len = [&](int b) { return (indptr[b + 1] - indptr[b] - 1) * kPage + last[b]; };
    const size_t pairs = (size_t)B * Hkv;
    struct SegRef { int64_t w; int idx; size_t pair; };
    std::vector<int32_t> desc;
    std::vector<SegRef> refs;
    std::vector<int> nc;
    // appends segment {b, kvh, pages [p0, p1) of sequence b} to workgroup w, whose page list starts
    // at page-table position wbeg (relative to kv_indptr[0]); false when w is full
    auto add_segment = [&](int64_t w, int64_t wbeg, int b, int kvh, int p0, int p1) {
        int32_t* d = &desc[(size_t)w * kBalDescInts];
        if (d[0] == seg_cap) return false;
        int32_t* sg = d + 8 + kSegInts * d[0];
        const int np = indptr[b + 1] - indptr[b];
        const int64_t pos = indptr[b] - jbase + p0;
        sg[0] = b;
        sg[1] = kvh;
        sg[2] = (int)(pos - wbeg);
        sg[3] = p1 - p0;
        sg[4] = p0 * kPage;
        sg[5] = p1 == np ? seq_len(b) : p1 * kPage;
        sg[6] = (int)pos;
        sg[7] = -1;
        const size_t pr = (size_t)b * Hkv + kvh;
        refs.push_back({w, d[0], pr});
        ++nc[pr];
        ++d[0];
        return true;
    };
    if (grouped) {
        int64_t NG = std::min<int64_t>(W / Hkv, std::max<int64_t>(1, nnz));
        for (;;) {
            W = NG * Hkv;
            desc.assign((size_t)W * kBalDescInts, 0);
            refs.clear();
            nc.assign(pairs, 0);
            bool ok = true;
            int b = 0;
            for (int64_t g = 0; g < NG && ok; ++g) {
                const int64_t lo = nnz * g / NG, hi = nnz * (g + 1) / NG;
                if (hi - lo > kRangeMax) { ok = false; break; }
                while (b < B && indptr[b + 1] - jbase <= lo) ++b;   // first sequence reaching past lo
                for (int bb = b; bb < B && indptr[bb] - jbase < hi && ok; ++bb) {
                    const int64_t s0 = std::max<int64_t>(lo, indptr[bb] - jbase);
                    const int64_t s1 = std::min<int64_t>(hi, indptr[bb + 1] - jbase);
                    if (s1 <= s0) continue;   // an empty sequence
                    const int p0 = (int)(s0 - (indptr[bb] - jbase)), p1 = (int)(s1 - (indptr[bb] - jbase));
                    for (int kvh = 0; kvh < Hkv && ok; ++kvh) ok = add_segment(g * Hkv + kvh, lo, bb, kvh, p0, p1);
                }
            }
            if (ok) break;
            if (NG >= std::max<int64_t>(1, nnz)) return fail(PDATTN_ERR_INVALID_ARGUMENT, "cannot partition the batch");
            NG = std::min<int64_t>(std::max<int64_t>(1, nnz), NG * 2);
        }
        pl->P = (int)((nnz + W / Hkv - 1) / (W / Hkv));   // pages per range
        pl->ngroups = (int)(W / Hkv);
        pl->pair = pair;   // (W = NG Hkv is even: plan workgroups 2 x and 2 x + 1 share range g)
    }
    for (; !grouped;) {
        desc.assign((size_t)W * kBalDescInts, 0);
        refs.clear();
        nc.assign(pairs, 0);
        bool ok = true;
        int64_t w = 0, u = 0;
        int64_t wbeg = 0, wend = U / W;
        for (int b = 0; b < B && ok; ++b) {
            const int np = indptr[b + 1] - indptr[b];
            for (int pa = 0; pa < np && ok; pa += P) {
                const int pn = std::min(P, np - pa);
                for (int kvh = 0; kvh < Hkv && ok; ++kvh) {
                    for (int done = 0; done < pn;) {
                        while (u >= wend) {
                            ++w;
                            wbeg = wend;
                            wend = U * (w + 1) / W;
                        }
                        if (wend - wbeg > kRangeMax) { ok = false; break; }
                        const int take = (int)std::min<int64_t>(pn - done, wend - u);
                        int32_t* d = &desc[(size_t)w * kBalDescInts];
                        if (d[0] == seg_cap) { ok = false; break; }
                        int32_t* sg = d + 8 + kSegInts * d[0];
                        const int p0 = pa + done, p1 = pa + done + take;
                        sg[0] = b;
                        sg[1] = kvh;
                        sg[2] = (int)(u - wbeg);
                        sg[3] = take;
                        sg[4] = p0 * kPage;
                        sg[5] = p1 == np ? seq_len(b) : p1 * kPage;
                        sg[6] = indptr[b] - pl->jbase + p0;
                        sg[7] = -1;
                        const size_t pr = (size_t)b * Hkv + kvh;
                        refs.push_back({w, d[0], pr});
                        ++nc[pr];
                        ++d[0];
                        u += take;
                        done += take;
                    }
                }
            }
        }
        if (ok) break;
        if (W >= U) return fail(PDATTN_ERR_INVALID_ARGUMENT, "cannot partition the batch");
        W = std::min<int64_t>(U, W * 2);
    }

    // partial slots and merge list: pairs in (b, kv head) order, contributors in unit order.
    // Packed, contributor k of a listed pair is slot slot0 + k with the pairs' slots consecutive;
    // laid out by entry (cmax = the most contributors of a listed pair), contributor k of entry e
    // is slot e * cmax + k, which the merge can address before it has read the entry. The entry
    // layout is used unless it would take more than twice the packed slots (a few long pairs among
    // many short ones).
    std::vector<int32_t> slot0(pairs, -1), list;
    int slots = 0, split = 0, mx = 1, cmax = 0;
    auto need_slots = [&](size_t pr) { return nc[pr] > 1 || (merge_all && nc[pr] > 0); };
    for (int b = 0; b < B; ++b)
        for (int kvh = 0; kvh < Hkv; ++kvh) {
            const size_t pr = (size_t)b * Hkv + kvh;
            if (nc[pr] > 1) ++split;
            mx = std::max(mx, nc[pr]);
            if (need_slots(pr)) {
                slot0[pr] = slots;
                slots += nc[pr];
                cmax = std::max(cmax, nc[pr]);
                list.insert(list.end(), {b, kvh, slot0[pr], nc[pr]});
            } else if (nc[pr] == 0) {
                list.insert(list.end(), {b, kvh, 0, 0});   // empty sequence: extras only, or 0 / -inf
            }
        }
    const int64_t n_list = (int64_t)(list.size() / 4);
    if (cmax > 0 && n_list * cmax <= 2 * (int64_t)slots + 64) {
        for (int64_t e = 0; e < n_list; ++e) {
            const size_t pr = (size_t)list[4 * e] * Hkv + list[4 * e + 1];
            list[4 * e + 2] = (int32_t)(e * cmax);
            if (slot0[pr] >= 0) slot0[pr] = (int32_t)(e * cmax);
        }
        slots = (int)(n_list * cmax);
    } else {
        cmax = 0;
    }
    std::vector<int> seen(pairs, 0);
    for (const SegRef& rf : refs) {
        int32_t* sg = &desc[(size_t)rf.w * kBalDescInts + 8 + kSegInts * rf.idx];
        const int k = seen[rf.pair]++;
        if (need_slots(rf.pair)) sg[7] = slot0[rf.pair] + k;
    }

    pl->W = (int)W;
    pl->split_pairs = split;
    pl->max_contrib = mx;
    pl->n_entries = (int)(list.size() / 4);
    pl->n_slots = slots;
    pl->cmax = cmax;
    pl->segments = (int)refs.size();
    for (int64_t w = 0; w < W; ++w) desc[(size_t)w * kBalDescInts + 1] = pl->tag;
    pl->host_blob = desc;
    pl->host_blob.insert(pl->host_blob.end(), {pl->tag, pl->n_entries, cmax, 0});   // list header
    pl->host_blob.insert(pl->host_blob.end(), list.begin(), list.end());

    size_t off = 0;
    pl->off_desc = off;  off += align_up(sizeof(int32_t) * desc.size());
    pl->off_list = off;  off += align_up(sizeof(int32_t) * (4 + list.size()));
    pl->off_plse = off;  off += align_up(sizeof(float) * std::max(1, slots) * G);
    pl->off_po = off;    off += align_up(sizeof(float) * std::max(1, slots) * G * kHeadDim);
    pl->ws_bytes = off;
    pl->blob_bytes = sizeof(int32_t) * pl->host_blob.size();
    return PDATTN_OK;
}

void free_plan_storage(pdattn_plan* pl) {
    if (pl) res_forget(pl->id);
    if (pl && pl->pinned) {
        (void)hipHostFree(pl->pinned);
        pl->pinned = nullptr;
    }
}

// Bytes of a plan's schedule in its workspace (descriptors and merge list; the partial slots
// after them are scratch of each run).
size_t schedule_bytes(const pdattn_plan* pl) { return pl->off_plse - pl->off_desc; }

int upload_plan(pdattn_plan* pl, void* ws, size_t bytes, hipStream_t s) {
    if (!ws) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null workspace");
    if (bytes < pl->ws_bytes)
        return fail(PDATTN_ERR_WORKSPACE, "workspace holds %zu bytes, plan needs %zu", bytes, pl->ws_bytes);
    char* base = static_cast<char*>(ws);
    const size_t desc_bytes = sizeof(int32_t) * (size_t)pl->W * kBalDescInts;
    if (pl->blob_bytes && !pl->pinned) {
        // pinned staging copy, made once: the copies below are stream-ordered and asynchronous
        hipError_t e = hipHostMalloc(&pl->pinned, pl->blob_bytes, hipHostMallocDefault);
        if (e != hipSuccess) return hip_fail(e, "hipHostMalloc(plan)");
        std::memcpy(pl->pinned, pl->host_blob.data(), pl->blob_bytes);
    }
    if (pl->blob_bytes) {
        PD_HIP(hipMemcpyAsync(base + pl->off_desc, pl->pinned, desc_bytes, hipMemcpyHostToDevice, s));
        PD_HIP(hipMemcpyAsync(base + pl->off_list, static_cast<char*>(pl->pinned) + desc_bytes,
                              sizeof(int32_t) * 4 * (1 + pl->n_entries), hipMemcpyHostToDevice, s));
    }
    res_claim(base + pl->off_desc, schedule_bytes(pl), pl->id);
    return PDATTN_OK;
}

// The argument block of a plan's decode launch (its workspace already checked).
BalArgs bal_args(const pdattn_plan* pl, const void* q, const void* k, const void* v,
                 const int32_t* indices, float sm_scale, void* out, float* lse, char* base) {
    BalArgs a;
    a.q = static_cast<const _Float16*>(q);
    a.k = static_cast<const uint8_t*>(k);
    a.v = static_cast<const uint8_t*>(v);
    a.kv_indices = indices + pl->jbase;
    a.out = static_cast<_Float16*>(out);
    a.lse = lse;
    a.desc = reinterpret_cast<const int32_t*>(base + pl->off_desc);
    a.part_o = reinterpret_cast<float*>(base + pl->off_po);
    a.part_lse = reinterpret_cast<float*>(base + pl->off_plse);
    a.B = pl->B;
    a.Hq = pl->Hq;
    a.Hkv = pl->Hkv;
    a.W = pl->W;
    a.scale_log2 = sm_scale * 1.4426950408889634f;
    a.part_stride = 0;   // the planner's slot-major partials
    a.ngroups = pl->ngroups;
    a.nnz = pl->nnz;
    a.tag = pl->tag;
    a.qrow_b = pl->ngroups > 0 && pl->B == 1 ? 0 : -1;
    return a;
}

// Balanced decode launch, then (when the plan lists any) the merge launch. With `join`, the
// stream waits for that event between the two (the extra partials come from another stream).
// decode = false: the decode workgroups ran elsewhere (the fused cascade step); merge only.
// merge = false: the decode launch only (pdattn_plan_run_part).
int run_plan(const pdattn_plan* pl, const void* q, const void* k, const void* v,
             const int32_t* indptr, const int32_t* indices, const int32_t* last, float sm_scale,
             void* out, float* lse, void* ws, size_t bytes, hipStream_t s,
             const float* extra_o = nullptr, const float* extra_lse = nullptr, int n_extra = 0,
             hipEvent_t join = nullptr, bool decode = true, bool merge = true) {
    if (!ws || !res_holds(static_cast<char*>(ws) + pl->off_desc, schedule_bytes(pl), pl->id))
        return fail(PDATTN_ERR_NOT_READY,
                    "plan's schedule is not in this workspace (never uploaded there, or overwritten "
                    "since by another upload or launch): upload it again");
    if (bytes < pl->ws_bytes)
        return fail(PDATTN_ERR_WORKSPACE, "workspace holds %zu bytes, plan needs %zu", bytes, pl->ws_bytes);
    if (pl->B == 0) return PDATTN_OK;
    if (!out || !lse || !q || !indptr || !last || (pl->U > 0 && (!k || !v || !indices)))
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "null device pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "q / k_cache / v_cache / out must be 16-byte aligned");
    if (!std::isfinite(sm_scale)) return fail(PDATTN_ERR_INVALID_ARGUMENT, "sm_scale is not finite");
    char* base = static_cast<char*>(ws);
    float* part_lse = reinterpret_cast<float*>(base + pl->off_plse);
    float* part_o = reinterpret_cast<float*>(base + pl->off_po);
    res_written(part_lse, pl->ws_bytes - pl->off_plse, pl->id);
    res_written_outputs(out, lse, (size_t)pl->B * pl->Hq);
    if (pl->U > 0 && decode) {
        const BalArgs a = bal_args(pl, q, k, v, indices, sm_scale, out, lse, base);
        if (pl->pair) PD_HIP(launch_decode_pair(a, pl->G, s));
        else PD_HIP(launch_decode_balanced(a, pl->G, s));
    }
    if (join) PD_HIP(hipStreamWaitEvent(s, join, 0));
    if (pl->n_entries && merge) {
        MergeArgs m;
        m.list = reinterpret_cast<const int32_t*>(base + pl->off_list);
        m.part_o = part_o;
        m.part_lse = part_lse;
        m.extra_o = extra_o;
        m.extra_lse = extra_lse;
        m.out = static_cast<_Float16*>(out);
        m.lse = lse;
        m.B = pl->B;
        m.Hq = pl->Hq;
        m.Hkv = pl->Hkv;
        m.G = pl->G;
        m.n_extra = n_extra;
        m.cmax = pl->cmax;
        m.n_slots = pl->n_slots;
        m.tag = pl->tag;
        PD_HIP(launch_merge_split(m, pl->n_entries, s));
    }
    return PDATTN_OK;
}


// Nodes of the shared-prefix structure of a batch and the first suffix page of every sequence.
// tree = false: the reference's rule (plan_cascade, 01_decode_attention.cu:656-701): one node,
// the longest prefix every sequence shares (shared_prefix_pages), used if it holds at least
// min_prefix tokens. tree = true: a prefix tree. A group of sequences that share the page at
// position p0 extends its node while every member holds the same page and keeps a page of its
// own after it; a node of at least min_prefix tokens is kept, and the group splits by the page
// that follows, each subgroup of two or more sequences descending. A group whose shared run is
// shorter than min_prefix stops there (its pages are decoded with each member's suffix).
void build_cascade_nodes(const int32_t* indptr, const int32_t* indices, int B, int min_prefix,
                         bool tree, std::vector<CascadeNode>& nodes, std::vector<int32_t>& seqs,
                         std::vector<int>& suffix_start) {
    suffix_start.assign(std::max(1, B), 0);
    auto np = [&](int b) { return indptr[b + 1] - indptr[b]; };
    auto page = [&](int b, int p) { return indices[indptr[b] + p]; };
    if (!tree) {
        const int P = B > 0 ? pdattn_shared_prefix_pages(indptr, indices, B) : 0;
        if (P > 0 && P * kPage >= min_prefix) {
            CascadeNode n;
            n.p0 = 0;
            n.p1 = P;
            n.jpos = indptr[0];
            n.seq_off = 0;
            n.ns = B;
            nodes.push_back(n);
            for (int b = 0; b < B; ++b) seqs.push_back(b);
            for (int b = 0; b < B; ++b) suffix_start[b] = P;
        }
        return;
    }
    struct Work { std::vector<int> S; int p0, depth; };
    std::vector<Work> stack;
    // the root groups: sequences with two or more pages, by their first page
    std::map<int, std::vector<int>> roots;
    for (int b = 0; b < B; ++b)
        if (np(b) >= 2) roots[page(b, 0)].push_back(b);
    for (auto& kv : roots)
        if (kv.second.size() >= 2) stack.push_back({kv.second, 0, 0});
    while (!stack.empty()) {
        Work wk = std::move(stack.back());
        stack.pop_back();
        int p = wk.p0;
        for (;;) {
            bool ok = true;
            for (int b : wk.S)
                if (p >= np(b) - 1 || page(b, p) != page(wk.S[0], p)) { ok = false; break; }
            if (!ok) break;
            ++p;
        }
        if ((p - wk.p0) * kPage < min_prefix || p == wk.p0) continue;   // members keep start p0
        CascadeNode n;
        n.p0 = wk.p0;
        n.p1 = p;
        n.jpos = indptr[wk.S[0]] + wk.p0;
        n.depth = wk.depth;
        n.seq_off = (int)seqs.size();
        n.ns = (int)wk.S.size();
        nodes.push_back(n);
        seqs.insert(seqs.end(), wk.S.begin(), wk.S.end());
        std::map<int, std::vector<int>> sub;
        for (int b : wk.S) {
            suffix_start[b] = p;
            if (p < np(b) - 1) sub[page(b, p)].push_back(b);
        }
        for (auto& kv : sub)
            if (kv.second.size() >= 2) stack.push_back({kv.second, p, wk.depth + 1});
    }
}

int cascade_plan_create(const pdattn_decode_params* base, const int32_t* h_indptr,
                        const int32_t* h_indices, const int32_t* h_lens, const int32_t* d_indices,
                        int min_prefix, bool tree, pdattn_cascade_plan** plan) {
    if (!plan) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null plan output");
    *plan = nullptr;
    if (!base) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null base params");
    int G = 0;
    if (int st = check_heads(base->Hq, base->Hkv, &G)) return st;
    const int B = base->B;
    if (B < 0) return fail(PDATTN_ERR_INVALID_ARGUMENT, "B=%d is negative", B);
    if (base->kv_start != 0) return fail(PDATTN_ERR_INVALID_ARGUMENT, "cascade base must have kv_start = 0");
    if (B > 0 && (!h_indptr || !h_indices || !h_lens || !d_indices))
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "null host table / lens / device indices");
    if (B > 0 && (!base->q || !base->k_cache || !base->v_cache || !base->kv_indptr || !base->kv_indices ||
                  !base->kv_last_page_len))
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "null device pointer in base params");
    if (!std::isfinite(base->sm_scale)) return fail(PDATTN_ERR_INVALID_ARGUMENT, "sm_scale is not finite");
    // last-page lengths from the sequence lengths (ceil(L/16) pages each)
    std::vector<int32_t> last(std::max(1, B), 0);
    for (int b = 0; b < B; ++b) {
        const int np = h_indptr[b + 1] - h_indptr[b];
        if (np < 0) return fail(PDATTN_ERR_PAGE_TABLE, "indptr not monotone at %d", b);
        if (h_lens[b] < 0 || (h_lens[b] + kPage - 1) / kPage != np)
            return fail(PDATTN_ERR_PAGE_TABLE, "lens[%d]=%d does not match its %d pages", b, h_lens[b], np);
        last[b] = np > 0 ? h_lens[b] - (np - 1) * kPage : 0;
    }
    DeviceFacts f;
    if (int st = device_facts(&f)) return st;

    pdattn_cascade_plan* cp = new pdattn_cascade_plan();
    cp->base = *base;
    cp->d_indices = d_indices;
    std::vector<int32_t> seqs;
    std::vector<int> start;
    build_cascade_nodes(h_indptr, h_indices, B, min_prefix, tree, cp->nodes, seqs, start);
    cp->use = cp->nodes.empty() ? 0 : 1;
    int st = PDATTN_OK;
    if (!cp->use) {
        if (!tree) {
            const int P = B > 0 ? pdattn_shared_prefix_pages(h_indptr, h_indices, B) : 0;
            if (P < 0) { delete cp; return -P; }
            cp->Lp = P * kPage;
        }
        st = build_balanced_plan(h_indptr, last.data(), B, base->Hq, base->Hkv, 0, 0, false, &cp->sk);
        cp->off_sk = 0;
        cp->ws_bytes = cp->sk.ws_bytes;
    } else {
        // compacted suffix page table: pages start[b].. of every sequence
        std::vector<int32_t> sind(B + 1, 0);
        std::vector<int32_t> sidx;
        for (int b = 0; b < B; ++b) {
            for (int i = h_indptr[b] + start[b]; i < h_indptr[b + 1]; ++i) sidx.push_back(h_indices[i]);
            sind[b + 1] = (int32_t)sidx.size();
        }
        st = build_balanced_plan(sind.data(), last.data(), B, base->Hq, base->Hkv, 0, 0, true, &cp->sk);
        // The prefix work of every node goes into one launch (nodes of different depths write
        // different partial columns, so they are independent). Fused step (default where two of
        // its workgroups fit on a CU): about one prefix workgroup per CU, beside the suffix
        // decode's one. Separate prefix launch: enough workgroups to fill every CU slot. Chunk
        // tokens ctok (a multiple of 64 in [256, 8192]) such that the sum over nodes of query
        // groups x Hkv x ceil(tokens / ctok) is about that target. Partial columns: one range per
        // depth, as wide as its node with the most chunks.
        // Fused: a workgroup with few query rows is cheap (its waves hold one tile or none), so
        // the target grows as the work-weighted rows per group fall below the 128 a workgroup
        // holds: about one prefix workgroup per CU at 128 rows, up to three at 43 or fewer
        // (measured best for 256-row single-level and 32-row tree nodes).
        cp->mode = f.occ_step[G] >= 2 ? PDATTN_CASCADE_FUSED : PDATTN_CASCADE_SERIAL;
        int depths = 0;
        for (const CascadeNode& n : cp->nodes) depths = std::max(depths, n.depth + 1);
        std::vector<int> depth_cols(depths, 0);
        double units = 0, row_units = 0;
        for (CascadeNode& n : cp->nodes) {
            const int Lp = (n.p1 - n.p0) * kPage;
            n.qgroups = (n.ns * G + prefix_rows_per_workgroup() - 1) / prefix_rows_per_workgroup();
            units += (double)n.qgroups * base->Hkv * Lp;
            row_units += (double)n.ns * G * base->Hkv * Lp;
        }
        const double grp_rows = units > 0 ? row_units / units : prefix_rows_per_workgroup();
        const double scale = std::min(3.0, std::max(1.0, prefix_rows_per_workgroup() / grp_rows));
        const int target = cp->mode == PDATTN_CASCADE_FUSED ? (int)(f.cus * scale)
                                                             : f.cus * std::max(1, f.occ_prefix[G]);
        int ctok = (int)(units / target);
        ctok = std::min(std::max((ctok + 63) / 64 * 64, 256), 8192);
        for (CascadeNode& n : cp->nodes) {
            const int Lp = (n.p1 - n.p0) * kPage;
            n.ctok = std::min(ctok, (Lp + 63) / 64 * 64);
            n.nchunks = (Lp + n.ctok - 1) / n.ctok;
            depth_cols[n.depth] = std::max(depth_cols[n.depth], n.nchunks);
        }
        std::vector<int> col_of_depth(depths + 1, 0);
        for (int d = 0; d < depths; ++d) col_of_depth[d + 1] = col_of_depth[d] + depth_cols[d];
        for (CascadeNode& n : cp->nodes) n.col0 = col_of_depth[n.depth];
        cp->n_extra = col_of_depth.back();
        cp->levels = depths;
        cp->Lp = (cp->nodes[0].p1 - cp->nodes[0].p0) * kPage;
        // the item list (items of depth 0 first), each item carrying its node's fields
        std::vector<int32_t> items;
        cp->level_items.assign(depths, 0);
        for (int d = 0; d < depths; ++d)
            for (size_t k = 0; k < cp->nodes.size(); ++k) {
                const CascadeNode& n = cp->nodes[k];
                if (n.depth != d) continue;
                // The query groups of one chunk read the same keys. Workgroups are dispatched to
                // the XCDs round-robin by block index, so items kXcds apart run on the same XCD:
                // chunks go in runs of kXcds per query group, and a chunk's second read hits that
                // XCD's L2 (measured: fused cascade step 51.4 -> 47.9 us at 64 x (8192 + 512)).
                for (int c0 = 0; c0 < n.nchunks; c0 += kXcds)
                    for (int qg = 0; qg < n.qgroups; ++qg)
                        for (int c = c0; c < std::min(c0 + kXcds, n.nchunks); ++c) {
                            items.insert(items.end(), {n.jpos, n.seq_off, n.ns, (n.p1 - n.p0) * kPage,
                                                       n.ctok, n.col0, c, qg});
                            ++cp->level_items[d];
                        }
            }
        cp->n_items = (int)(items.size() / 8);
        cp->n_suffix_idx = (int)sidx.size();
        cp->blob = sind;
        cp->blob.insert(cp->blob.end(), sidx.begin(), sidx.end());
        cp->blob.insert(cp->blob.end(), seqs.begin(), seqs.end());
        cp->n_seqs = (int)seqs.size();
        cp->blob.insert(cp->blob.end(), items.begin(), items.end());
        const size_t rows = (size_t)B * base->Hq;
        size_t off = 0;
        cp->off_ppo = off;   off += align_up(rows * cp->n_extra * kHeadDim * sizeof(float));
        cp->off_pplse = off; off += align_up(rows * cp->n_extra * sizeof(float));
        cp->off_blob = off;  off += align_up(cp->blob.size() * sizeof(int32_t));
        cp->off_sk = off;    off += cp->sk.ws_bytes;
        cp->ws_bytes = off;
    }
    if (st != PDATTN_OK) {
        pdattn_cascade_plan_destroy(cp);
        return st;
    }
    *plan = cp;
    return PDATTN_OK;
}

}  // namespace

extern "C" {

const char* pdattn_strerror(int status) {
    switch (status) {
        case PDATTN_OK: return "PDATTN_OK";
        case PDATTN_ERR_INVALID_ARGUMENT: return "PDATTN_ERR_INVALID_ARGUMENT";
        case PDATTN_ERR_UNSUPPORTED: return "PDATTN_ERR_UNSUPPORTED";
        case PDATTN_ERR_PAGE_TABLE: return "PDATTN_ERR_PAGE_TABLE";
        case PDATTN_ERR_WORKSPACE: return "PDATTN_ERR_WORKSPACE";
        case PDATTN_ERR_HIP: return "PDATTN_ERR_HIP";
        case PDATTN_ERR_NOT_READY: return "PDATTN_ERR_NOT_READY";
        default: return "PDATTN_ERR_UNKNOWN";
    }
}

const char* pdattn_last_error(void) { return g_last_error.c_str(); }

int pdattn_workspace_reserve(pdattn_workspace* ws, size_t bytes) {
    if (!ws) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null workspace");
    if (ws->base && ws->bytes >= bytes) return PDATTN_OK;
    if (ws->base && !ws->owned)
        return fail(PDATTN_ERR_WORKSPACE, "caller-provided workspace holds %zu bytes, %zu needed", ws->bytes, bytes);
    if (ws->base) {
        PD_HIP(hipDeviceSynchronize());
        res_written(ws->base, ws->bytes);   // freed: what was uploaded there is gone
        PD_HIP(hipFree(ws->base));
        ws->base = nullptr;
        ws->bytes = 0;
    }
    void* p = nullptr;
    PD_HIP(hipMalloc(&p, std::max<size_t>(bytes, kAlign)));
    ws->base = p;
    ws->bytes = std::max<size_t>(bytes, kAlign);
    ws->owned = 1;
    return PDATTN_OK;
}

void pdattn_workspace_release(pdattn_workspace* ws) {
    if (!ws) return;
    if (ws->base && ws->owned) {
        (void)hipDeviceSynchronize();
        res_written(ws->base, ws->bytes);
        (void)hipFree(ws->base);
    }
    ws->base = nullptr;
    ws->bytes = 0;
    ws->owned = 0;
}

int pdattn_check_page_table(const int32_t* h_indptr, const int32_t* h_indices, const int32_t* h_last,
                            int B, int64_t num_pages) {
    if (B < 0 || num_pages < 0) return fail(PDATTN_ERR_INVALID_ARGUMENT, "B=%d num_pages=%lld", B, (long long)num_pages);
    if (!h_indptr) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null kv_indptr");
    if (int st = check_host_table(h_indptr, h_last, B)) return st;
    if (h_indptr[B] > h_indptr[0] && !h_indices) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null kv_indices");
    for (int b = 0; b < B; ++b)
        for (int j = h_indptr[b]; j < h_indptr[b + 1]; ++j)
            if (h_indices[j] < 0 || h_indices[j] >= num_pages)
                return fail(PDATTN_ERR_PAGE_TABLE, "kv_indices[%d] = %d (page %d of sequence %d) outside [0, %lld)",
                            j, h_indices[j], j - h_indptr[b], b, (long long)num_pages);
    return PDATTN_OK;
}

int pdattn_plan_chunks(int G, int variant, int B, int Hkv, int max_len, int force_chunks,
                       int* num_chunks, int* chunk_tokens) {
    if (!num_chunks || !chunk_tokens) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null output");
    if (!valid_group(G)) return fail(PDATTN_ERR_UNSUPPORTED, "GQA group size %d not in {1,2,4,8}", G);
    if (variant < 0 || variant > 3) return fail(PDATTN_ERR_INVALID_ARGUMENT, "variant %d not in 0..3", variant);
    if (B < 0 || Hkv <= 0 || max_len < 0 || force_chunks < 0)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "B=%d Hkv=%d max_len=%d force=%d", B, Hkv, max_len, force_chunks);
    int chunks;
    if (force_chunks > 0) {
        chunks = force_chunks;
    } else {
        DeviceFacts f;
        if (int st = device_facts(&f)) return st;
        // One workgroup per CU, rounded down, and chunks of at least 256 tokens. The 4-wave
        // kernel's occupancy would allow more per CU, but more, shorter chunks measured slower
        // (1x32K: 32 chunks 33.2 us, 94 chunks 39.2 us; 8x8K: 4 chunks 53.3 us, 12 chunks 57.4 us).
        const int64_t resident = (int64_t)f.cus;
        const int64_t want = std::max<int64_t>(1, resident / std::max<int64_t>(1, (int64_t)B * Hkv));
        const int64_t cap = std::max<int64_t>(1, ((int64_t)max_len + 255) / 256);
        chunks = (int)std::min(want, cap);
    }
    const int per = (max_len + chunks - 1) / chunks;
    int tokens = (per + kPage - 1) / kPage * kPage;  // whole pages per chunk
    if (tokens < kPage) tokens = kPage;
    *chunk_tokens = tokens;
    *num_chunks = std::max(1, (max_len + tokens - 1) / tokens);
    return PDATTN_OK;
}

// The uniform split's partial launch. Its items (pair, chunk) run on the balanced workgroup body,
// several per workgroup so that the grid is about one workgroup per CU, with the segment
// descriptors built in the kernel (so that the call needs only the device page table, as the
// reference's does). A chunk spans at most ceil(chunk_tokens / 16) + 1 pages; one whose pages do
// not fit the body's LDS page list (kRangeMax) runs on the one-chunk-per-workgroup kernel. With
// `out` set (one chunk per sequence, nothing to merge), out / lse are written instead of partials.
static int launch_uniform_split(const PartialArgs& a, int G, hipStream_t s) {
    const int64_t ppi = ((int64_t)a.chunk_tokens + kPage - 1) / kPage + 1;
    if (ppi > kRangeMax) {
        PD_HIP(launch_decode_partial(a, G, s));
        return PDATTN_OK;
    }
    DeviceFacts f;
    if (int st = device_facts(&f)) return st;
    const int64_t n_items = (int64_t)a.num_chunks * a.B * a.Hkv;
    if (n_items > (int64_t)1 << 30) return fail(PDATTN_ERR_INVALID_ARGUMENT, "too many chunks");
    // at G = 8 the kernel's compact layout holds kStepSegMax segments, two workgroups per CU
    const bool wide = G > 4;
    const int64_t slots = (int64_t)f.cus * (wide ? 2 : 1);
    int64_t per = (n_items + slots - 1) / slots;
    per = std::max<int64_t>(1, std::min<int64_t>({per, (int64_t)(wide ? kStepSegMax : kSegMax), kRangeMax / ppi}));
    UniArgs u;
    BalArgs& d = u.d;
    d.q = a.q;
    d.k = a.k;
    d.v = a.v;
    d.kv_indices = a.kv_indices;
    d.out = a.out;
    d.lse = a.lse;
    d.desc = nullptr;
    d.part_o = a.part_o;
    d.part_lse = a.part_lse;
    d.B = a.B;
    d.Hq = a.Hq;
    d.Hkv = a.Hkv;
    d.W = (int)((n_items + per - 1) / per);
    d.scale_log2 = a.scale_log2;
    d.part_stride = a.part_stride;
    d.ngroups = 0;
    d.nnz = 0;
    d.tag = 0;   // (descriptors built in the kernel: no tag to check)
    u.kv_indptr = a.kv_indptr;
    u.kv_last = a.kv_last;
    u.kv_start = a.kv_start;
    u.chunk_tokens = a.chunk_tokens;
    u.num_chunks = a.num_chunks;
    u.chunk_base = a.chunk_base;
    u.n_items = (int)n_items;
    u.per_wg = (int)per;
    PD_HIP(launch_decode_uniform(u, G, s));
    return PDATTN_OK;
}

int pdattn_decode_partial(const pdattn_decode_params* p, int G, int variant, void* stream) {
    if (variant < 0 || variant > 3) return fail(PDATTN_ERR_INVALID_ARGUMENT, "variant %d not in 0..3", variant);
    if (int st = check_decode_params(p, G)) return st;
    if (p->B == 0) return PDATTN_OK;
    if (!p->part_o || !p->part_lse) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null part_o / part_lse");
    const size_t slots = (size_t)p->B * p->Hq * p->part_stride;
    res_written(p->part_o, slots * kHeadDim * sizeof(float));
    res_written(p->part_lse, slots * sizeof(float));
    return launch_uniform_split(to_partial_args(p), G, static_cast<hipStream_t>(stream));
}

int pdattn_merge_states(const float* part_o, const float* part_lse, void* out, float* lse_out,
                        int rows, int num_chunks, void* stream) {
    if (rows < 0 || num_chunks < 1) return fail(PDATTN_ERR_INVALID_ARGUMENT, "rows=%d num_chunks=%d", rows, num_chunks);
    if (rows == 0) return PDATTN_OK;
    if (!part_o || !part_lse || !out || !lse_out) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null pointer");
    res_written_outputs(out, lse_out, (size_t)rows);
    PD_HIP(launch_merge_states(part_o, part_lse, static_cast<_Float16*>(out), lse_out, rows, num_chunks,
                               static_cast<hipStream_t>(stream)));
    return PDATTN_OK;
}

size_t pdattn_decode_workspace_size(int B, int Hq, int part_stride) {
    if (B < 0 || Hq < 0 || part_stride < 0) return 0;
    const size_t rows = (size_t)B * Hq * part_stride;
    return align_up(rows * kHeadDim * sizeof(float)) + align_up(rows * sizeof(float));
}

int pdattn_workspace_partials(const pdattn_workspace* ws, int B, int Hq, int part_stride,
                              float** part_o, float** part_lse) {
    if (!ws || !part_o || !part_lse) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null pointer");
    const size_t need = pdattn_decode_workspace_size(B, Hq, part_stride);
    if (!ws->base || ws->bytes < need) return fail(PDATTN_ERR_WORKSPACE, "workspace smaller than %zu bytes", need);
    const size_t rows = (size_t)B * Hq * part_stride;
    *part_o = static_cast<float*>(ws->base);
    *part_lse = reinterpret_cast<float*>(static_cast<char*>(ws->base) + align_up(rows * kHeadDim * sizeof(float)));
    return PDATTN_OK;
}

}  // extern "C"

namespace pdattn {

int decode_attention_check(const pdattn_decode_params* p, int G, int variant, const void* out,
                           const float* lse) {
    if (variant < 0 || variant > 3) return fail(PDATTN_ERR_INVALID_ARGUMENT, "variant %d not in 0..3", variant);
    if (int st = check_decode_params(p, G)) return st;
    if (p->B == 0) return PDATTN_OK;
    if (!out || !lse) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null out / lse");
    // the merge reads part_stride slots per row: every one of them must be written by this call
    if (p->chunk_base != 0 || p->part_stride != p->num_chunks)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "decode_attention needs chunk_base = 0 and part_stride = num_chunks");
    return PDATTN_OK;
}

int decode_attention_launch(const pdattn_decode_params* p, int G, void* out, float* lse, float* part_o,
                            float* part_lse, hipStream_t s) {
    res_written_outputs(out, lse, (size_t)p->B * p->Hq);
    pdattn_decode_params q = *p;
    q.part_o = part_o;
    q.part_lse = part_lse;
    PartialArgs a = to_partial_args(&q);
    if (p->num_chunks == 1) {
        // one chunk per sequence: the partial kernel writes the result (merge_states of a single
        // state returns it unchanged), and the merge launch is skipped
        a.out = static_cast<_Float16*>(out);
        a.lse = lse;
        return launch_uniform_split(a, G, s);
    }
    if (int st = launch_uniform_split(a, G, s)) return st;
    PD_HIP(launch_merge_states(part_o, part_lse, static_cast<_Float16*>(out), lse, p->B * p->Hq,
                               p->part_stride, s));
    return PDATTN_OK;
}

int report_error(int status, const char* what) { return fail(status, "%s", what); }

}  // namespace pdattn

extern "C" {

int pdattn_decode_attention(const pdattn_decode_params* p, int G, int variant, void* out,
                            float* lse, pdattn_workspace* ws, void* stream) {
    if (int st = decode_attention_check(p, G, variant, out, lse)) return st;
    if (p->B == 0) return PDATTN_OK;
    const size_t need = pdattn_decode_workspace_size(p->B, p->Hq, p->part_stride);
    if (int st = ensure_ws(ws, need)) return st;
    float *part_o = nullptr, *part_lse = nullptr;
    if (int st = pdattn_workspace_partials(ws, p->B, p->Hq, p->part_stride, &part_o, &part_lse)) return st;
    res_written(ws->base, need);   // the partials: any schedule uploaded there is overwritten
    return decode_attention_launch(p, G, out, lse, part_o, part_lse, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

// Layout of the device-range decode (pdattn_decode_attention_balanced): the grid, ranges and the
// workspace, or use_uniform when the batch is past the kernel's staging (kDevMaxB sequences).
struct DevLayout {
    bool use_uniform = false;
    int W = 0, NG = 0;
    int64_t span = 0;
    size_t off_prefix = 0, off_plse = 0, off_po = 0, bytes = 0;
};

int dev_layout(const pdattn_decode_params* p, int G, DevLayout* L) {
    *L = DevLayout();
    if (p->B > kDevMaxB) {
        L->use_uniform = true;
        L->bytes = pdattn_decode_workspace_size(p->B, p->Hq, p->part_stride);
        return PDATTN_OK;
    }
    DeviceFacts f;
    if (int st = device_facts(&f)) return st;
    // one workgroup per CU (two at G = 8, as the plan path), whole groups of Hkv; more ranges if a
    // range could hold more pages than the kernel stages (kRangeMax): every sequence attends at
    // most ceil(span / 16) + 1 pages
    L->span = (int64_t)p->num_chunks * p->chunk_tokens;
    const int64_t per_seq = L->span / kPage + 2;
    const int64_t bound = (int64_t)p->B * per_seq;
    int64_t NG = std::max<int64_t>(1, (int64_t)f.cus * (G > 4 ? 2 : 1) / p->Hkv);
    NG = std::max<int64_t>(NG, (bound + kRangeMax - 1) / kRangeMax);
    if (NG * p->Hkv > (1 << 24)) return fail(PDATTN_ERR_INVALID_ARGUMENT, "too many ranges");
    L->NG = (int)NG;
    L->W = (int)(NG * p->Hkv);
    const size_t slots = (size_t)2 * L->W * G;
    size_t off = 0;
    L->off_prefix = off; off += align_up(sizeof(int32_t) * (p->B + 1));
    L->off_plse = off;   off += align_up(sizeof(float) * slots);
    L->off_po = off;     off += align_up(sizeof(float) * slots * kHeadDim);
    L->bytes = off;
    return PDATTN_OK;
}

}  // namespace

extern "C" {

size_t pdattn_decode_balanced_workspace_size(const pdattn_decode_params* p, int G) {
    if (!p || check_decode_params(p, G) != PDATTN_OK) return 0;
    if (p->B == 0) return 0;
    DevLayout L;
    if (dev_layout(p, G, &L) != PDATTN_OK) return 0;
    return L.bytes;
}

int pdattn_decode_attention_balanced(const pdattn_decode_params* p, int G, int variant, void* out,
                                     float* lse, pdattn_workspace* ws, void* stream) {
    if (variant < 0 || variant > 3) return fail(PDATTN_ERR_INVALID_ARGUMENT, "variant %d not in 0..3", variant);
    if (int st = check_decode_params(p, G)) return st;
    if (p->B == 0) return PDATTN_OK;
    if (!out || !lse) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null out / lse");
    DevLayout L;
    if (int st = dev_layout(p, G, &L)) return st;
    if (L.use_uniform) return pdattn_decode_attention(p, G, variant, out, lse, ws, stream);
    if (int st = ensure_ws(ws, L.bytes)) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* base = static_cast<char*>(ws->base);
    res_written(base, L.bytes);
    res_written_outputs(out, lse, (size_t)p->B * p->Hq);
    DevArgs a;
    BalArgs& d = a.d;
    d.q = static_cast<const _Float16*>(p->q);
    d.k = static_cast<const uint8_t*>(p->k_cache);
    d.v = static_cast<const uint8_t*>(p->v_cache);
    d.kv_indices = p->kv_indices;
    d.out = static_cast<_Float16*>(out);
    d.lse = lse;
    d.desc = nullptr;
    d.part_o = reinterpret_cast<float*>(base + L.off_po);
    d.part_lse = reinterpret_cast<float*>(base + L.off_plse);
    d.B = p->B;
    d.Hq = p->Hq;
    d.Hkv = p->Hkv;
    d.W = L.W;
    d.scale_log2 = p->sm_scale * 1.4426950408889634f;
    d.part_stride = 0;
    d.ngroups = L.NG;
    d.nnz = 0;
    d.tag = 0;   // (descriptors built in the kernel: no tag to check)
    a.kv_indptr = p->kv_indptr;
    a.kv_last = p->kv_last_page_len;
    a.prefix = reinterpret_cast<int32_t*>(base + L.off_prefix);
    a.span = L.span;
    a.kv_start = p->kv_start;
    PD_HIP(launch_decode_ranges(a, G, s));
    DevMergeArgs m;
    m.prefix = a.prefix;
    m.part_o = d.part_o;
    m.part_lse = d.part_lse;
    m.out = d.out;
    m.lse = lse;
    m.B = p->B;
    m.Hq = p->Hq;
    m.Hkv = p->Hkv;
    m.G = G;
    m.ngroups = L.NG;
    PD_HIP(launch_merge_ranges(m, s));
    return PDATTN_OK;
}

int pdattn_plan_create(const int32_t* h_kv_indptr, const int32_t* h_kv_last_page_len, int B,
                       int Hq, int Hkv, int force_workgroups, int chunk_pages, pdattn_plan** plan) {
    if (!plan) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null plan output");
    *plan = nullptr;
    if (B > 0 && !h_kv_indptr) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null kv_indptr");
    pdattn_plan* pl = new pdattn_plan();
    int st = build_balanced_plan(h_kv_indptr, h_kv_last_page_len, B, Hq, Hkv, force_workgroups,
                                 chunk_pages, false, pl, 0, true);
    if (st == PDATTN_OK && pl->pair && pl->n_entries > 0) {
        // The paired plan's ranges are half as long, so it splits this batch's sequences over
        // twice as many workgroups: the merge's fan-in doubles, which costs more than the paired
        // kernel gains (1x32K: 28.3 -> 30.8 us back to back). One kv head per workgroup instead.
        free_plan_storage(pl);
        delete pl;
        pl = new pdattn_plan();
        st = build_balanced_plan(h_kv_indptr, h_kv_last_page_len, B, Hq, Hkv, force_workgroups,
                                 chunk_pages, false, pl);
    }
    if (st != PDATTN_OK) {
        free_plan_storage(pl);
        delete pl;
        return st;
    }
    *plan = pl;
    return PDATTN_OK;
}

int pdattn_plan_get_info(const pdattn_plan* pl, pdattn_plan_info* info) {
    if (!pl || !info) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null pointer");
    info->workgroups = pl->W;
    info->pairs = pl->B * pl->Hkv;
    info->split_pairs = pl->split_pairs;
    info->max_contributors = pl->max_contrib;
    info->units = pl->U;
    info->workspace_bytes = pl->ws_bytes;
    info->chunk_pages = pl->P;
    info->segments = pl->segments;
    info->merge_entries = pl->n_entries;
    info->paired = pl->pair ? 1 : 0;
    info->schedule_ints = (int)pl->host_blob.size();
    return PDATTN_OK;
}

int pdattn_plan_get_schedule(const pdattn_plan* pl, int32_t* out, size_t count) {
    if (!pl || !out) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null pointer");
    if (count < pl->host_blob.size())
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "schedule holds %zu ints, %zu given", pl->host_blob.size(), count);
    std::memcpy(out, pl->host_blob.data(), sizeof(int32_t) * pl->host_blob.size());
    return PDATTN_OK;
}

size_t pdattn_plan_workspace_size(const pdattn_plan* pl) { return pl ? pl->ws_bytes : 0; }

int pdattn_plan_upload(pdattn_plan* pl, void* workspace, size_t bytes, void* stream) {
    if (!pl) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null plan");
    return upload_plan(pl, workspace, bytes, static_cast<hipStream_t>(stream));
}

int pdattn_plan_run(const pdattn_plan* pl, const void* q, const void* k_cache, const void* v_cache,
                    const int32_t* kv_indptr, const int32_t* kv_indices,
                    const int32_t* kv_last_page_len, float sm_scale, void* out, float* lse,
                    void* workspace, size_t bytes, void* stream) {
    if (!pl) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null plan");
    return run_plan(pl, q, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, sm_scale,
                    out, lse, workspace, bytes, static_cast<hipStream_t>(stream));
}

int pdattn_plan_run_part(const pdattn_plan* pl, const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* kv_indptr, const int32_t* kv_indices,
                         const int32_t* kv_last_page_len, float sm_scale, void* out, float* lse,
                         void* workspace, size_t bytes, void* stream, int parts) {
    if (!pl) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null plan");
    if (parts < PDATTN_RUN_DECODE || parts > PDATTN_RUN_ALL)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "parts=%d not in 1..3", parts);
    return run_plan(pl, q, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, sm_scale,
                    out, lse, workspace, bytes, static_cast<hipStream_t>(stream), nullptr, nullptr, 0,
                    nullptr, (parts & PDATTN_RUN_DECODE) != 0, (parts & PDATTN_RUN_MERGE) != 0);
}

void pdattn_plan_destroy(pdattn_plan* pl) {
    if (!pl) return;
    free_plan_storage(pl);
    delete pl;
}

int pdattn_shared_prefix_pages(const int32_t* h_indptr, const int32_t* h_indices, int B) {
    if (B < 0 || !h_indptr || (B > 0 && !h_indices)) return -fail(PDATTN_ERR_INVALID_ARGUMENT, "null table or B < 0");
    for (int b = 0; b < B; ++b)
        if (h_indptr[b + 1] < h_indptr[b]) return -fail(PDATTN_ERR_PAGE_TABLE, "indptr not monotone at %d", b);
    if (B < 2) return 0;
    // longest P with indices[indptr[b] + i] equal across b for i < P, P <= npages_b - 1 for all b
    for (int P = 0;; ++P) {
        for (int b = 0; b < B; ++b)
            if (P >= h_indptr[b + 1] - h_indptr[b] - 1) return P;
        const int pg = h_indices[h_indptr[0] + P];
        for (int b = 1; b < B; ++b)
            if (h_indices[h_indptr[b] + P] != pg) return P;
    }
}

int pdattn_cascade_prefix(const pdattn_prefix_params* p, void* stream) {
    if (!p) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null params");
    int G = 0;
    if (int st = check_heads(p->Hq, p->Hkv, &G)) return st;
    if (p->B < 0 || p->prefix_len < 0) return fail(PDATTN_ERR_INVALID_ARGUMENT, "B / prefix_len negative");
    if (p->B == 0 || p->prefix_len == 0) return PDATTN_OK;
    if (!p->q || !p->k_cache || !p->v_cache || !p->prefix_pages || !p->part_o || !p->part_lse)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "null device pointer");
    if (!aligned16(p->q) || !aligned16(p->k_cache) || !aligned16(p->v_cache) || !aligned16(p->part_o))
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "q / caches / part_o must be 16-byte aligned");
    if (p->chunk_tokens < kPage || p->chunk_tokens % kPage || p->chunk_tokens > 8192)
        return fail(PDATTN_ERR_UNSUPPORTED, "chunk_tokens=%d must be a multiple of 16 in [16, 8192]", p->chunk_tokens);
    const int nchunks = (p->prefix_len + p->chunk_tokens - 1) / p->chunk_tokens;
    if (p->part_stride < nchunks)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "part_stride=%d < %d prefix chunks", p->part_stride, nchunks);
    PrefixArgs a;
    a.q = static_cast<const _Float16*>(p->q);
    a.k = static_cast<const uint8_t*>(p->k_cache);
    a.v = static_cast<const uint8_t*>(p->v_cache);
    a.prefix_pages = p->prefix_pages;
    a.part_o = p->part_o;
    a.part_lse = p->part_lse;
    a.B = p->B;
    a.Hq = p->Hq;
    a.Hkv = p->Hkv;
    a.prefix_len = p->prefix_len;
    a.chunk_tokens = p->chunk_tokens;
    a.part_stride = p->part_stride;
    a.num_chunks = nchunks;
    a.seqs = nullptr;
    a.items = nullptr;
    a.ns = p->B;
    a.col0 = 0;
    a.scale_log2 = p->sm_scale * 1.4426950408889634f;
    const size_t slots = (size_t)p->B * p->Hq * p->part_stride;
    res_written(p->part_o, slots * kHeadDim * sizeof(float));
    res_written(p->part_lse, slots * sizeof(float));
    PD_HIP(launch_cascade_prefix(a, G, static_cast<hipStream_t>(stream)));
    return PDATTN_OK;
}

int pdattn_cascade_plan_create(const pdattn_decode_params* base, const int32_t* h_indptr,
                               const int32_t* h_indices, const int32_t* h_lens,
                               const int32_t* d_indices, int min_prefix,
                               pdattn_cascade_plan** plan) {
    return cascade_plan_create(base, h_indptr, h_indices, h_lens, d_indices, min_prefix, false, plan);
}

int pdattn_cascade_tree_plan_create(const pdattn_decode_params* base, const int32_t* h_indptr,
                                    const int32_t* h_indices, const int32_t* h_lens,
                                    const int32_t* d_indices, int min_prefix,
                                    pdattn_cascade_plan** plan) {
    return cascade_plan_create(base, h_indptr, h_indices, h_lens, d_indices, min_prefix, true, plan);
}

int pdattn_cascade_plan_get_info(const pdattn_cascade_plan* cp, pdattn_cascade_info* info) {
    if (!cp || !info) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null pointer");
    info->use = cp->use;
    info->prefix_tokens = cp->Lp;
    info->prefix_chunks = cp->n_extra;
    info->prefix_workgroups = cp->n_items * cp->base.Hkv;
    info->suffix_workgroups = cp->sk.W;
    info->workspace_bytes = cp->ws_bytes;
    info->nodes = (int)cp->nodes.size();
    info->levels = cp->levels;
    info->mode = cp->mode;
    return PDATTN_OK;
}

int pdattn_cascade_decode(pdattn_cascade_plan* cp, void* out, float* lse, pdattn_workspace* ws,
                          void* stream) {
    if (!cp) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null plan");
    if (cp->base.B == 0) return PDATTN_OK;
    if (!out || !lse) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null out / lse");
    if (int st = ensure_ws(ws, cp->ws_bytes)) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* base = static_cast<char*>(ws->base);
    const pdattn_decode_params& p = cp->base;
    float* ppo = reinterpret_cast<float*>(base + cp->off_ppo);
    float* pplse = reinterpret_cast<float*>(base + cp->off_pplse);
    const size_t n_lse = (size_t)p.B * p.Hq * cp->n_extra;
    const size_t blob_bytes = cp->blob.size() * sizeof(int32_t);
    const bool resident =
        res_holds(base + cp->off_sk + cp->sk.off_desc, schedule_bytes(&cp->sk), cp->sk.id) &&
        (!cp->use || (res_holds(base + cp->off_blob, blob_bytes, cp->id) &&
                      (n_lse == 0 || res_holds(pplse, n_lse * sizeof(float), cp->id))));
    if (!resident) {
        // first call with this workspace, or another call has written over the plan's part of it
        if (cp->use && !cp->pinned) {
            hipError_t e = hipHostMalloc(&cp->pinned, cp->blob.size() * sizeof(int32_t), hipHostMallocDefault);
            if (e != hipSuccess) return hip_fail(e, "hipHostMalloc(cascade plan)");
            std::memcpy(cp->pinned, cp->blob.data(), cp->blob.size() * sizeof(int32_t));
        }
        if (cp->use) {
            PD_HIP(hipMemcpyAsync(base + cp->off_blob, cp->pinned, blob_bytes, hipMemcpyHostToDevice, s));
            res_claim(base + cp->off_blob, blob_bytes, cp->id);
            // partial columns no node writes for a row stay empty (lse = -inf) for good
            PD_HIP(launch_fill_i32(reinterpret_cast<int32_t*>(pplse), (int32_t)0xff800000u, n_lse, s));
            res_claim(pplse, n_lse * sizeof(float), cp->id);
        }
        if (int st = upload_plan(&cp->sk, base + cp->off_sk, cp->sk.ws_bytes, s)) return st;
    }
    // the prefix pass writes the node columns of the partials (the -inf columns stay as filled)
    res_written(ppo, cp->off_pplse - cp->off_ppo, cp->id);
    if (!cp->use)
        return run_plan(&cp->sk, p.q, p.k_cache, p.v_cache, p.kv_indptr, p.kv_indices,
                        p.kv_last_page_len, p.sm_scale, out, lse, base + cp->off_sk, cp->sk.ws_bytes, s);
    const int32_t* sind = reinterpret_cast<const int32_t*>(base + cp->off_blob);
    const int32_t* sidx = sind + (p.B + 1);
    const int32_t* dseqs = sidx + cp->n_suffix_idx;
    const int32_t* ditems = dseqs + cp->n_seqs;
    // the prefix pass over every node's items (one workgroup per item and kv head)
    PrefixArgs a;
    a.q = static_cast<const _Float16*>(p.q);
    a.k = static_cast<const uint8_t*>(p.k_cache);
    a.v = static_cast<const uint8_t*>(p.v_cache);
    a.prefix_pages = cp->d_indices;
    a.seqs = dseqs;
    a.items = ditems;
    a.part_o = ppo;
    a.part_lse = pplse;
    a.B = p.B;
    a.Hq = p.Hq;
    a.Hkv = p.Hkv;
    a.prefix_len = 0;
    a.chunk_tokens = 0;
    a.part_stride = cp->n_extra;
    a.num_chunks = cp->n_items;
    a.ns = 0;
    a.col0 = 0;
    a.scale_log2 = p.sm_scale * 1.4426950408889634f;
    char* skb = base + cp->off_sk;
    if (cp->mode == PDATTN_CASCADE_FUSED) {
        // one launch: the suffix decode's workgroups, then the prefix workgroups beside them
        if (!res_holds(skb + cp->sk.off_desc, schedule_bytes(&cp->sk), cp->sk.id))
            return fail(PDATTN_ERR_NOT_READY, "suffix plan was not uploaded into this workspace");
        StepArgs sa;
        sa.d = bal_args(&cp->sk, p.q, p.k_cache, p.v_cache, sidx, p.sm_scale, out, lse, skb);
        sa.p = a;
        sa.n_dec = cp->sk.U > 0 ? cp->sk.W : 0;
        sa.n_pre = cp->n_items * p.Hkv;
        PD_HIP(launch_cascade_step(sa, p.Hq / p.Hkv, s));
        return run_plan(&cp->sk, p.q, p.k_cache, p.v_cache, sind, sidx, p.kv_last_page_len, p.sm_scale,
                        out, lse, skb, cp->sk.ws_bytes, s, ppo, pplse, cp->n_extra, nullptr, false);
    }
    // Separate launches. Two streams: the prefix launch runs on the plan's second stream while
    // the suffix decode runs on `s`; `s` waits for it before the merge, so the step stays one
    // fork / join (graph-capturable).
    const bool two = cp->mode == PDATTN_CASCADE_TWO_STREAMS;
    hipStream_t ps = s;
    if (two) {
        if (!cp->aux) {
            PD_HIP(hipStreamCreateWithFlags(&cp->aux, hipStreamNonBlocking));
            PD_HIP(hipEventCreateWithFlags(&cp->ev_fork, hipEventDisableTiming));
            PD_HIP(hipEventCreateWithFlags(&cp->ev_join, hipEventDisableTiming));
        }
        PD_HIP(hipEventRecord(cp->ev_fork, s));
        PD_HIP(hipStreamWaitEvent(cp->aux, cp->ev_fork, 0));
        ps = cp->aux;
    }
    PD_HIP(launch_cascade_prefix(a, p.Hq / p.Hkv, ps));
    if (two) PD_HIP(hipEventRecord(cp->ev_join, ps));
    return run_plan(&cp->sk, p.q, p.k_cache, p.v_cache, sind, sidx, p.kv_last_page_len, p.sm_scale,
                    out, lse, skb, cp->sk.ws_bytes, s, ppo, pplse, cp->n_extra,
                    two ? cp->ev_join : nullptr);
}

int pdattn_cascade_set_mode(pdattn_cascade_plan* cp, int mode) {
    if (!cp) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null plan");
    if (mode != PDATTN_CASCADE_FUSED && mode != PDATTN_CASCADE_SERIAL && mode != PDATTN_CASCADE_TWO_STREAMS)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "unknown cascade mode %d", mode);
    if (mode == PDATTN_CASCADE_FUSED) {
        DeviceFacts f;
        if (int st = device_facts(&f)) return st;
        const int G = cp->base.Hkv > 0 ? cp->base.Hq / cp->base.Hkv : 1;
        if (G < 1 || G > 8 || f.occ_step[G] < 2)
            return fail(PDATTN_ERR_UNSUPPORTED, "the fused cascade step does not fit two workgroups per CU at G=%d", G);
    }
    cp->mode = mode;
    return PDATTN_OK;
}

void pdattn_cascade_plan_destroy(pdattn_cascade_plan* cp) {
    if (!cp) return;
    if (cp->aux) (void)hipStreamSynchronize(cp->aux);
    if (cp->ev_fork) (void)hipEventDestroy(cp->ev_fork);
    if (cp->ev_join) (void)hipEventDestroy(cp->ev_join);
    if (cp->aux) (void)hipStreamDestroy(cp->aux);
    free_plan_storage(&cp->sk);
    res_forget(cp->id);
    if (cp->pinned) (void)hipHostFree(cp->pinned);
    delete cp;
}

int pdattn_append_kv(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                     const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* batch_idx,
                     const int32_t* positions, int n, int B, int Hkv, int32_t* n_invalid,
                     void* stream) {
    if (n < 0 || B < 0 || Hkv <= 0)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "n=%d B=%d Hkv=%d", n, B, Hkv);
    if (n == 0) return PDATTN_OK;
    if (!k_new || !v_new || !k_cache || !v_cache || !kv_indptr || !kv_indices || !batch_idx || !positions)
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "null device pointer");
    if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(k_cache) || !aligned16(v_cache))
        return fail(PDATTN_ERR_INVALID_ARGUMENT, "K/V inputs and caches must be 16-byte aligned");
    DeviceFacts f;
    if (int st = device_facts(&f)) return st;
    AppendArgs a;
    a.k_new = k_new;
    a.v_new = v_new;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.kv_indptr = kv_indptr;
    a.kv_indices = kv_indices;
    a.batch_idx = batch_idx;
    a.positions = positions;
    a.n_invalid = n_invalid;
    a.n = n;
    a.B = B;
    a.Hkv = Hkv;
    PD_HIP(launch_append_kv(a, f.cus, static_cast<hipStream_t>(stream)));
    return PDATTN_OK;
}

int pdattn_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream) {
    if (!buf || !sink || bytes % 16) return fail(PDATTN_ERR_INVALID_ARGUMENT, "buf/sink null or bytes %% 16 != 0");
    if (bytes == 0) return PDATTN_OK;
    DeviceFacts f;
    if (int st = device_facts(&f)) return st;
    PD_HIP(launch_stream_read(buf, bytes, sink, f.cus, static_cast<hipStream_t>(stream)));
    return PDATTN_OK;
}

int pdattn_flush_cache(void* buf, size_t bytes, void* stream) {
    if (!buf || bytes % 16) return fail(PDATTN_ERR_INVALID_ARGUMENT, "buf null or bytes %% 16 != 0");
    if (bytes == 0) return PDATTN_OK;
    DeviceFacts f;
    if (int st = device_facts(&f)) return st;
    PD_HIP(launch_flush(buf, bytes, f.cus * 16, static_cast<hipStream_t>(stream)));
    return PDATTN_OK;
}

int pdattn_get_device_info(pdattn_device_info* info) {
    if (!info) return fail(PDATTN_ERR_INVALID_ARGUMENT, "null info");
    DeviceFacts f;
    if (int st = device_facts(&f)) return st;
    info->compute_units = f.cus;
    info->decode_wg_per_cu = f.occ_balanced[4];
    info->prefix_wg_per_cu = f.occ_prefix[4];
    snprintf(info->arch, sizeof info->arch, "%s", f.arch);
    return PDATTN_OK;
}

}  // extern "C"
