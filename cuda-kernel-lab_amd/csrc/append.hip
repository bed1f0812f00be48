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
// Byte work, HBM-bound. A workgroup of 256 threads takes several tokens, 4096 16-byte pieces of
// K and V in all (16 tokens at Hkv = 8, 16 pieces per thread). One thread per token resolves the
// token's page slot from the page table into LDS; meanwhile every thread has already issued the
// loads of its pieces, which do not depend on the page table, so the table's dependent loads
// overlap the data loads, and after one barrier the pieces are stored. A token's Hkv rows are
// contiguous both in the input [n, Hkv, 128] and in its page slot ([16, Hkv, 128] per page), so
// reads and writes are coalesced runs. A token whose position lies outside its sequence's pages
// is not written; it is counted in *n_invalid.
#include <algorithm>

#include "pdattn_internal.h"

namespace pdattn {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kAppendThreads = 256;
constexpr int kAppendPieces = 16;                                  // 16-byte pieces per thread per pass
constexpr int kAppendMaxTokens = kAppendThreads * kAppendPieces / 32;   // at Hkv = 1

// the most tokens a workgroup takes: as many as fill one pass of kAppendPieces pieces per thread
inline int append_max_tokens_per_wg(int Hkv) {
    const int ppt = 2 * Hkv * (kHeadDim / 8);
    return ppt >= kAppendThreads * kAppendPieces ? 1 : kAppendThreads * kAppendPieces / ppt;
}

__global__ __launch_bounds__(kAppendThreads) void append_kv_kernel(AppendArgs a) {
    __shared__ long long s_dst[kAppendMaxTokens];   // first piece of the token's slot row, or -1
    const int tid = threadIdx.x;
    const int row_pieces = a.Hkv * (kHeadDim / 8);  // 16-byte pieces of one token's K (or V)
    const int ppt = 2 * row_pieces;                 // per token: K then V
    const int tpb = a.tpb;
    const size_t t0 = (size_t)blockIdx.x * tpb;
    const int ntok = (int)min((size_t)tpb, (size_t)a.n - t0);

    if (tpb == 1) {   // one token (a decode step's few tokens): its slot is uniform, no LDS hand-off
        const int b = a.batch_idx[t0], pos = a.positions[t0];
        const bool ok_b = b >= 0 && b < a.B;
        const int pb = ok_b ? a.kv_indptr[b] : 0, np = ok_b ? a.kv_indptr[b + 1] - pb : 0;
        if (!ok_b || pos < 0 || pos >= np * kPage) {
            if (tid == 0 && a.n_invalid) atomicAdd(a.n_invalid, 1);
            return;
        }
        const size_t page = (size_t)(uint32_t)a.kv_indices[pb + pos / kPage];
        const size_t dst = (page * kPage + pos % kPage) * row_pieces;
        const u32x4* kn = reinterpret_cast<const u32x4*>(a.k_new) + t0 * row_pieces;
        const u32x4* vn = reinterpret_cast<const u32x4*>(a.v_new) + t0 * row_pieces;
        u32x4* kc = reinterpret_cast<u32x4*>(a.k_cache) + dst;
        u32x4* vc = reinterpret_cast<u32x4*>(a.v_cache) + dst;
        for (int pc = tid; pc < ppt; pc += kAppendThreads) {
            if (pc < row_pieces) kc[pc] = kn[pc];
            else vc[pc - row_pieces] = vn[pc - row_pieces];
        }
        return;
    }

    if (tid < ntok) {
        const size_t t = t0 + tid;
        const int b = a.batch_idx[t], pos = a.positions[t];
        const bool ok_b = b >= 0 && b < a.B;
        const int pb = ok_b ? a.kv_indptr[b] : 0, np = ok_b ? a.kv_indptr[b + 1] - pb : 0;
        long long dst = -1;
        if (ok_b && pos >= 0 && pos < np * kPage) {
            const size_t page = (size_t)(uint32_t)a.kv_indices[pb + pos / kPage];
            dst = (long long)((page * kPage + pos % kPage) * row_pieces);
        } else if (a.n_invalid) {
            atomicAdd(a.n_invalid, 1);
        }
        s_dst[tid] = dst;
    }

    const u32x4* kn = reinterpret_cast<const u32x4*>(a.k_new) + t0 * row_pieces;
    const u32x4* vn = reinterpret_cast<const u32x4*>(a.v_new) + t0 * row_pieces;
    u32x4* kc = reinterpret_cast<u32x4*>(a.k_cache);
    u32x4* vc = reinterpret_cast<u32x4*>(a.v_cache);
    const int total = ntok * ppt;
    for (int base = 0; base < tpb * ppt; base += kAppendThreads * kAppendPieces) {   // uniform
        u32x4 val[kAppendPieces];
#pragma unroll
        for (int u = 0; u < kAppendPieces; ++u) {
            const int idx = base + u * kAppendThreads + tid;
            if (idx < total) {
                const int tok = idx / ppt, pc = idx % ppt;
                val[u] = pc < row_pieces ? kn[(size_t)tok * row_pieces + pc]
                                         : vn[(size_t)tok * row_pieces + pc - row_pieces];
            }
        }
        __syncthreads();   // the slots in s_dst
#pragma unroll
        for (int u = 0; u < kAppendPieces; ++u) {
            const int idx = base + u * kAppendThreads + tid;
            if (idx < total) {
                const int tok = idx / ppt, pc = idx % ppt;
                const long long dst = s_dst[tok];
                if (dst >= 0) {
                    if (pc < row_pieces) kc[dst + pc] = val[u];
                    else vc[dst + pc - row_pieces] = val[u];
                }
            }
        }
    }
}

}  // namespace

// Tokens per workgroup: enough workgroups for every CU first (a decode step's few tokens get one
// each), then up to one full pass per thread (a prefill's many tokens).
hipError_t launch_append_kv(const AppendArgs& args, int cus, hipStream_t s) {
    if (args.n <= 0) return hipSuccess;
    AppendArgs a = args;
    a.tpb = std::max(1, std::min(append_max_tokens_per_wg(a.Hkv), a.n / std::max(1, cus)));
    const size_t grid = ((size_t)a.n + a.tpb - 1) / a.tpb;
    append_kv_kernel<<<(unsigned)grid, kAppendThreads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace pdattn
