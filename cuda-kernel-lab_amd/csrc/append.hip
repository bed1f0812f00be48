// append.hip -- paged KV append: the step before decode that writes new tokens' K/V into the
// paged caches.
//
// Layout of the caches and the page table as in the decode path (qilem/cuda-kernel-lab,
// 01_decode_attention.cu:5-9, 112; FlashInfer's page-table convention): element (page, slot,
// kvh, d) at ((page*16 + slot)*Hkv + kvh)*128 + d. The page table already describes the caches
// after the append (the caller allocates pages and sets kv_indptr / kv_last_page_len first, as
// with FlashInfer's append_paged_kv_cache); token t, at position pos[t] of sequence b[t], goes to
// page kv_indices[kv_indptr[b] + pos / 16], slot pos % 16.
//
// Byte work, HBM-bound. A workgroup of 256 threads takes 256 / (2 * Hkv * 16) tokens (one token
// at Hkv = 8; a token's pieces are spread over several passes when Hkv > 8): every thread moves
// one 16-byte piece of a K or V row per pass, and the threads of one token read its page-table
// entries at the same addresses (one fetch each). A token's Hkv rows are contiguous both in the
// input [n, Hkv, 128] and in its page slot ([16, Hkv, 128] per page), so reads and writes are
// coalesced runs. A token whose position lies outside its sequence's pages is not written; it is
// counted in *n_invalid.
#include "pdattn_internal.h"

namespace pdattn {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kAppendThreads = 256;

__global__ __launch_bounds__(kAppendThreads) void append_kv_kernel(AppendArgs a) {
    const int row_pieces = a.Hkv * (kHeadDim / 8);            // 16-byte pieces of one cache row set
    const int ppt = 2 * row_pieces;                          // per token: K then V
    const int tpb = ppt >= kAppendThreads ? 1 : kAppendThreads / ppt;
    const size_t t0 = (size_t)blockIdx.x * tpb;
    for (int idx = threadIdx.x; idx < tpb * ppt; idx += kAppendThreads) {
        const size_t t = t0 + idx / ppt;
        if (t >= (size_t)a.n) break;
        const int pc = idx % ppt;
        const bool is_v = pc >= row_pieces;
        const int pr = is_v ? pc - row_pieces : pc;         // = kvh * 16 + piece within the row
        const int b = a.batch_idx[t], pos = a.positions[t];
        const bool ok_b = b >= 0 && b < a.B;
        const int pb = ok_b ? a.kv_indptr[b] : 0, np = ok_b ? a.kv_indptr[b + 1] - pb : 0;
        if (!ok_b || pos < 0 || pos >= np * kPage) {
            if (pc == 0 && a.n_invalid) atomicAdd(a.n_invalid, 1);
            continue;
        }
        const size_t page = (size_t)(uint32_t)a.kv_indices[pb + pos / kPage];
        const size_t dst = (page * kPage + pos % kPage) * row_pieces + pr;
        const u32x4* src = reinterpret_cast<const u32x4*>(is_v ? a.v_new : a.k_new) + t * row_pieces + pr;
        u32x4* cache = reinterpret_cast<u32x4*>(is_v ? a.v_cache : a.k_cache);
        cache[dst] = *src;
    }
}

}  // namespace

hipError_t launch_append_kv(const AppendArgs& a, int /*cus*/, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    const int ppt = 2 * a.Hkv * (kHeadDim / 8);
    const int tpb = ppt >= kAppendThreads ? 1 : kAppendThreads / ppt;
    const size_t grid = ((size_t)a.n + tpb - 1) / tpb;
    append_kv_kernel<<<(unsigned)grid, kAppendThreads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace pdattn
