// decode.hip -- paged split-KV GQA decode attention for gfx950 (CDNA4, wave64).
//
// What it computes (qilem/cuda-kernel-lab, 01_decode_attention.cu:76-255): for each sequence b,
// kv head kvh and each of the G query heads h sharing it, over a range of keys,
//   s_j = sm_scale * q_h . k_j,   o = sum_j softmax(s)_j v_j,   lse = ln sum_j exp(s_j)
// as a normalized partial (o, lse), then a log-sum-exp merge of the partials.
//
// How it maps to CDNA4:
//  * One workgroup body (balanced_body): 4 waves, one per SIMD and one workgroup per CU, walking
//    a list of segments (pieces of one sequence and kv head), each wave on every 4th page, with
//    one page ring across all of them. The plan/run path (decode_balanced_kernel) reads the list
//    from a host-built plan; the reference-shaped uniform split (decode_uniform_kernel) builds it
//    in the kernel from the device page table. A uniform chunk too long for the body's LDS page
//    list runs on decode_partial_kernel, one workgroup per (sequence, kv head, chunk).
//  * K and V rows go straight from HBM into VGPRs with 16-byte non-temporal loads: a 256-byte
//    row (128 fp16) is read by LPR lanes, so one wave-wide load instruction reads 64/LPR rows of
//    one page, each as whole 128-byte lines. No LDS staging is needed because every lane reads
//    only the bytes it computes with.
//  * Scores: each lane takes the fp16 dot product of its slice of q_h and k_j with
//    v_dot2_f32_f16 (fp32 accumulate), then the LPR lanes of a row sum with DPP row ops
//    (quad_perm, row_half_mirror, row_mirror), which leaves the score in every lane of the row.
//  * Every lane therefore owns whole keys: it keeps its own online-softmax state (max, sum,
//    output slice) over the keys it holds, so the PV product needs no cross-lane traffic. The
//    64/LPR independent states of a wave are merged once at the end, in the VALU (DPP row_ror and
//    v_permlane16/32_swap) or through LDS, and the waves of the workgroup through LDS.
//  * Softmax runs in base 2 on log2(e)-prescaled scores with v_exp_f32 / v_log_f32
//    (exp(x) = 2^(x log2 e)); the running output is rescaled only when some lane's max grows
//    (a wave-uniform branch), which after the first pages is rare.
//  * Prefetch: a two-page ring in VGPRs; the loads of the next page are issued before the
//    current page is computed.
//
// Lane geometry (both kernels), G = query heads per kv head: LPR = 16 lanes per 256-byte K/V row,
// 4 rows per wave-wide load, each lane holding 4 rows x 8 dims of a page (keeps the fp32 output
// state at 64 VGPRs at G = 8).
// Lane (r = lane / LPR, c = lane % LPR) holds rows i*RPI + r of each page and the 16-byte pieces
// kk*LPR + c (dims 8*(kk*LPR + c) .. +7), kk < PPL.
#include <math.h>

#include <algorithm>
#include <cstdlib>

#include "pdattn_internal.h"
#include "timeline.h"

PD_TIMELINE_TABLE(decode)

#include "prefix_body.h"

namespace pdattn {
namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;

// Compile-time shape of a decode kernel instance.
template <int G_, int LPR_, int NW_, int NBUF_>
struct Cfg {
    static constexpr int G = G_;                   // query heads per kv head
    static constexpr int LPR = LPR_;               // lanes per 256-byte K/V row (8 or 16)
    static constexpr int NW = NW_;                 // waves per workgroup
    static constexpr int NBUF = NBUF_;             // pages held in VGPRs per wave (NBUF-1 in flight)
    static constexpr int NT = NW * 64;
    static constexpr int RPI = 64 / LPR;           // rows per wave-wide load
    static constexpr int PPL = 16 / LPR;           // 16-byte pieces per lane per row
    static constexpr int RG = kPage / RPI;         // rows of each page held by one lane
    static constexpr int DPL = PPL * 8;            // head dims held by one lane
};

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the LPR lanes that share one K/V row (a DPP row is 16 lanes).
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror: the other quad of the 8-lane half row
    if constexpr (LPR == 16) v += dpp<0x140>(v);  // row_mirror: the other half row
    return v;
}

// row_sum of N independent values, one DPP step at a time across all of them (the same sums,
// bitwise: each value goes through the same sequence of adds).
template <int LPR, int N>
__device__ __forceinline__ void row_sum_all(float* v) {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] += dpp<0xB1>(v[j]);
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] += dpp<0x4E>(v[j]);
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] += dpp<0x141>(v[j]);
    if constexpr (LPR == 16) {
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] += dpp<0x140>(v[j]);
    }
}

// Combine of the 64/LPR row groups of a wave (lanes LPR apart hold the same head dims), leaving
// the result in every lane: row_ror:8 pairs the two groups of a 16-lane row (LPR = 8), then
// v_permlane16_swap / v_permlane32_swap pair whole 16-lane rows, all in the VALU. After
// swap(a, b) the two results hold, in every lane, the values of both rows of its pair (rows
// r and r^1 for the 16-lane swap, r and r^2 for the 32-lane swap), always in the same order, so
// r0 + r1 is bitwise the same in all lanes. The second operand is passed through an empty asm
// statement: given the same SSA value twice, the compiler treats the two results as equal and
// drops the second one. The statement is not volatile, so the many independent reductions of a
// merge can still be interleaved by the scheduler.
__device__ __forceinline__ unsigned opaque_copy(unsigned v) {
    asm("" : "+v"(v));
    return v;
}
template <bool ROWS32>
__device__ __forceinline__ void row_pair(float v, float& a, float& b) {
    const unsigned x = __builtin_bit_cast(unsigned, v);
    unsigned r0, r1;
    if constexpr (ROWS32) {
        const auto r = __builtin_amdgcn_permlane32_swap(x, opaque_copy(x), false, false);
        r0 = r[0]; r1 = r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(x, opaque_copy(x), false, false);
        r0 = r[0]; r1 = r[1];
    }
    a = __builtin_bit_cast(float, r0);
    b = __builtin_bit_cast(float, r1);
}

// Reinterprets one 32-bit word as two fp16. The word is taken by value: bit-casting an
// ext-vector element expression in place was observed to read element 0 for every index.
__device__ __forceinline__ f16x2 as_h2(uint32_t w) { return __builtin_bit_cast(f16x2, w); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

template <int LPR>
__device__ __forceinline__ float xgroup_sum(float v) {
    float a, b;
    if constexpr (LPR == 8) v += dpp<0x128>(v);   // row_ror:8
    row_pair<false>(v, a, b);
    row_pair<true>(a + b, a, b);
    return a + b;
}
template <int LPR>
__device__ __forceinline__ float xgroup_max(float v) {
    float a, b;
    if constexpr (LPR == 8) v = fmaxf(v, dpp<0x128>(v));
    row_pair<false>(v, a, b);
    row_pair<true>(fmaxf(a, b), a, b);
    return fmaxf(a, b);
}

template <class C>
struct WaveState {
    float m[C::G];                // running max, log2 units
    float l[C::G];                // running sum of 2^(x - m)
    float o[C::G][C::DPL];        // running unnormalized output slice
};

template <class C>
struct PageRegs {
    u32x4 k[C::RG][C::PPL];
    u32x4 v[C::RG][C::PPL];
};

template <int G, int NW>
struct Smem {
    float m[NW][G];
    float l[NW][G];
    float o[NW][G][kHeadDim];
    float fo[G][kHeadDim];    // combined, normalized output of the workgroup
    float flse[G];            // combined lse (natural log)
};

// A page of one kv head seen through a buffer resource: base = cache + page * page_bytes +
// kvh * 256, num_records = the bytes from there to the end of the page, so every lane's offset is
// in range. A padding slot of the ring uses num_records = 0: its loads return zeros without a
// memory access, while the ring still issues the same loads in every slot (exact wait counts).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const uint8_t* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, (int)bytes, 0x00020000);
}

template <class C>
__device__ __forceinline__ void load_page_rsrc(PageRegs<C>& pr, __amdgpu_buffer_rsrc_t rk,
                                               __amdgpu_buffer_rsrc_t rv, uint32_t lbase, uint32_t rstride) {
#pragma unroll
    for (int i = 0; i < C::RG; ++i)
#pragma unroll
        for (int kk = 0; kk < C::PPL; ++kk) {
            const int off = (int)(lbase + i * rstride + kk * (C::LPR * 16));
            // aux = 2: non-temporal (K/V bytes are read once)
            pr.k[i][kk] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 2);
            pr.v[i][kk] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 2);
        }
}

// One page: scores, online-softmax update, PV accumulation. tok0 is the (wave-uniform) token
// index of the page's first slot, and this lane's row of row group i is slot r + i * RPI; keys
// outside [tb, te) are masked. A masked key gets weight 0, and on a page that holds masked keys
// (the first or last page of a range) their V rows are zeroed as well, so that slots the cache
// never filled (NaN or Inf bit patterns in unused slots of a last page) cannot reach the output
// through 0 * v.
template <class C>
__device__ __forceinline__ void page_step(WaveState<C>& st, PageRegs<C>& pr,
                                          const f16x2 (&qv)[C::G][C::PPL][4], int tok0, int r,
                                          int tb, int te, float scale2) {
    using g = C;
    constexpr int G = C::G;
    const int tok_r = tok0 + r;
    if (tok0 < tb || tok0 + kPage > te) {   // wave-uniform: an edge page
#pragma unroll
        for (int i = 0; i < g::RG; ++i) {
            const int tok = tok_r + i * g::RPI;
            if (tok < tb || tok >= te) {
#pragma unroll
                for (int kk = 0; kk < g::PPL; ++kk) pr.v[i][kk] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    }
    // Scores: the lane's partial dot products of every (row, head) first, then each DPP step of
    // the row sums across all of them, so that every dependent DPP add has RG * G - 1 independent
    // instructions in front of it instead of a hazard stall (s_nop).
    float x[g::RG][G];
#pragma unroll
    for (int i = 0; i < g::RG; ++i)
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float acc = 0.f;
#pragma unroll
            for (int kk = 0; kk < g::PPL; ++kk)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc = __builtin_amdgcn_fdot2(qv[h][kk][e],
                                                 as_h2(pr.k[i][kk][e]), acc,
                                                 false);
            x[i][h] = acc;
        }
    row_sum_all<g::LPR, g::RG * G>(&x[0][0]);
#pragma unroll
    for (int i = 0; i < g::RG; ++i) {
        const int tok = tok_r + i * g::RPI;
        const bool ok = tok >= tb && tok < te;
#pragma unroll
        for (int h = 0; h < G; ++h) x[i][h] = ok ? x[i][h] * scale2 : -INFINITY;
    }
    float mn[G];
    bool grow = false;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float mt = x[0][h];
#pragma unroll
        for (int i = 1; i < g::RG; ++i) mt = fmaxf(mt, x[i][h]);
        mn[h] = fmaxf(st.m[h], mt);
        grow |= mn[h] > st.m[h];
    }
    if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float a = (mn[h] > st.m[h]) ? fast_exp2(st.m[h] - mn[h]) : 1.f;
            st.l[h] *= a;
#pragma unroll
            for (int d = 0; d < g::DPL; ++d) st.o[h][d] *= a;
            st.m[h] = mn[h];
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float ms = (st.m[h] == -INFINITY) ? 0.f : st.m[h];
#pragma unroll
        for (int i = 0; i < g::RG; ++i) {
            const float p = fast_exp2(x[i][h] - ms);
            st.l[h] += p;
#pragma unroll
            for (int kk = 0; kk < g::PPL; ++kk)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const f16x2 vv = as_h2(pr.v[i][kk][e]);
                    float* od = &st.o[h][kk * 8 + 2 * e];
                    od[0] = fmaf((float)vv[0], p, od[0]);
                    od[1] = fmaf((float)vv[1], p, od[1]);
                }
        }
    }
}

// Attention of the G query heads of (b, kvh) over keys [t0, t1) of one sequence. pages[i] is the
// physical page holding tokens [tok_base + 16 i, tok_base + 16 i + 16) (global memory or LDS).
// Leaves the normalized output in sm.fo and the lse in sm.flse (all threads of the workgroup
// must call it; it ends with a barrier).
template <class C>
__device__ __forceinline__ void process_range(Smem<C::G, C::NW>& sm, const _Float16* qrow, const uint8_t* kbase,
                              const uint8_t* vbase, const int32_t* pages, int tok_base, int t0, int t1,
                              int Hkv, int kvh, float scale2) {
    using g = C;
    constexpr int G = C::G, NW = C::NW, NBUF = C::NBUF;
    // the wave index is made wave-uniform explicitly: the page counts and buffer resources derived
    // from it must live in scalar registers (a non-uniform resource turns each load into a loop)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r = lane / g::LPR, c = lane % g::LPR;

    f16x2 qv[G][g::PPL][4];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int kk = 0; kk < g::PPL; ++kk) {
            const u32x4 raw =
                *reinterpret_cast<const u32x4*>(qrow + h * kHeadDim + (kk * g::LPR + c) * 8);
#pragma unroll
            for (int e = 0; e < 4; ++e) qv[h][kk][e] = as_h2(raw[e]);
        }

    WaveState<C> st;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        st.m[h] = -INFINITY;
        st.l[h] = 0.f;
#pragma unroll
        for (int d = 0; d < g::DPL; ++d) st.o[h][d] = 0.f;
    }

    if (t1 > t0) {
        const int pfirst = (t0 - tok_base) / kPage, plast = (t1 - 1 - tok_base) / kPage;
        const int npg = plast - pfirst + 1;
        const int nmine = npg > wave ? (npg - wave + NW - 1) / NW : 0;
        const uint32_t page_bytes = (uint32_t)(kPage * Hkv * 256);
        const uint32_t lbase = (uint32_t)(r * Hkv * 256 + c * 16);
        const uint32_t rstride = (uint32_t)(g::RPI * Hkv * 256);
        // slot j of the window: page j of it through a buffer resource over the rest of the page
        // (from this kv head's row), or, past the end, a zero-length resource whose loads return
        // zeros without a memory access, so every iteration issues the same loads (exact waits)
        // and no page is read twice
        auto issue = [&](PageRegs<C>& b, int pidv, int j, int cnt) {
            const uint8_t* kb = kbase;
            const uint8_t* vb = vbase;
            uint32_t nrec = 0;
            if (j < cnt) {
                const size_t off = (size_t)(uint32_t)__builtin_amdgcn_readlane(pidv, j) * page_bytes +
                                   (size_t)kvh * 256;
                kb += off;
                vb += off;
                nrec = page_bytes - (uint32_t)kvh * 256;
            }
            load_page_rsrc<C>(b, page_rsrc(kb, nrec), page_rsrc(vb, nrec), lbase, rstride);
        };
        for (int base = 0; base < nmine; base += 64) {
            const int cnt = min(64, nmine - base);
            // lane j holds the physical page of this wave's (base + j)-th page
            const int pidv = lane < cnt ? pages[pfirst + wave + NW * (base + lane)] : 0;
            // ring of NBUF pages in VGPRs: page i lives in buf[i % NBUF]; NBUF-1 are in flight
            // while one is computed
            PageRegs<C> buf[NBUF];
#pragma unroll
            for (int u = 0; u < NBUF - 1; ++u) issue(buf[u], pidv, u, cnt);
            for (int it = 0; it < cnt; it += NBUF) {
#pragma unroll
                for (int u = 0; u < NBUF; ++u) {
                    if (it + u >= cnt) break;
                    issue(buf[(u + NBUF - 1) % NBUF], pidv, it + u + NBUF - 1, cnt);
                    page_step<C>(st, buf[u], qv, tok_base + (pfirst + wave + NW * (base + it + u)) * kPage, r,
                                 t0, t1, scale2);
                }
            }
        }
    }

    // merge the 64/LPR row-group states of this wave (lanes LPR apart hold the same dims)
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float M = xgroup_max<g::LPR>(st.m[h]);
        const float a = (st.m[h] == -INFINITY) ? 0.f : fast_exp2(st.m[h] - M);
        st.l[h] = xgroup_sum<g::LPR>(st.l[h] * a);
#pragma unroll
        for (int d = 0; d < g::DPL; ++d) st.o[h][d] = xgroup_sum<g::LPR>(st.o[h][d] * a);
        st.m[h] = M;
    }
    if (lane < g::LPR) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int kk = 0; kk < g::PPL; ++kk)
#pragma unroll
                for (int e = 0; e < 8; ++e) sm.o[wave][h][(kk * g::LPR + c) * 8 + e] = st.o[h][kk * 8 + e];
        if (lane == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                sm.m[wave][h] = st.m[h];
                sm.l[wave][h] = st.l[h];
            }
        }
    }
    __syncthreads();
    for (int idx = tid; idx < G * kHeadDim; idx += NW * 64) {
        const int h = idx / kHeadDim, d = idx % kHeadDim;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, sm.m[w][h]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float a = (sm.m[w][h] == -INFINITY) ? 0.f : fast_exp2(sm.m[w][h] - M);
            L += a * sm.l[w][h];
            O += a * sm.o[w][h][d];
        }
        sm.fo[h][d] = L > 0.f ? O / L : 0.f;
        if (d == 0) sm.flse[h] = L > 0.f ? (M + fast_log2(L)) * kLn2 : -INFINITY;
    }
    __syncthreads();
}


// Kernel arguments of the balanced kernel read in place from the kernarg segment. The pointer is
// laundered through an empty asm statement at every use, so the compiler reloads those fields
// (scalar loads, cached) where they are needed instead of holding them in SGPRs across the page
// loop, where they would spill. The kernarg-segment intrinsic is only valid in the kernel body
// itself (in a called function it evaluates to null), so kargs() is called only from the kernel
// and the pointer is passed down to the (force-inlined) helpers.
typedef const __attribute__((address_space(4))) BalArgs* KArgPtr;
__device__ __forceinline__ KArgPtr kargs() {
    KArgPtr p = (KArgPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return p;
}

// ---- merging partial states ----------------------------------------------------------------
// Log-sum-exp merge of one row (128 dims) from partial states in a fixed order (merge_states,
// 01_decode_attention.cu:238-255), by one workgroup of kMergeThreads = 4 waves, with no LDS and no
// barrier. The sources are two lists, A then B (a pair's partial slots, then a cascade row's prefix
// partials): source k of a list has its lse at lse[k * stride] and its output row at
// o[k * stride * 128]. Wave w covers dims [32 w, 32 w + 32): lane 8 q + r holds the 4 dims
// 32 w + 4 q .. of sources r, r + 8, r + 16, ... of each list. The first 32 sources of both lists
// are loaded before any is waited for (one round trip), each lane folds its sources in order (A's,
// then B's), and the 8 source lanes of a quad are then combined by three DPP exchanges (lane
// distances 1, 2, then the other quad of the 8-lane half row): a fixed order, so the result is
// deterministic. keepA(k), evaluated after the loads, drops source k of A (a slot the decode launch
// did not write). The state is left in every lane: merged output acc / ws, lse m + ln ws.
constexpr int kMergeThreads = 256;
constexpr int kMergeU = 4;   // sources of a list per lane per round trip
struct MState {
    float m, ws;
    float4 acc;
};
struct MSrc {
    const float* lse;
    const float* o;
    size_t stride;
    int n;
};

template <int CTRL>
__device__ __forceinline__ void mstate_fold_dpp(MState& s) {
    const float m2 = dpp<CTRL>(s.m), w2 = dpp<CTRL>(s.ws);
    const float x2 = dpp<CTRL>(s.acc.x), y2 = dpp<CTRL>(s.acc.y);
    const float z2 = dpp<CTRL>(s.acc.z), u2 = dpp<CTRL>(s.acc.w);
    const float M = fmaxf(s.m, m2);
    const float s1 = (s.m == -INFINITY) ? 0.f : fast_exp2((s.m - M) * kLog2e);
    const float s2 = (m2 == -INFINITY) ? 0.f : fast_exp2((m2 - M) * kLog2e);
    s.ws = s.ws * s1 + w2 * s2;
    s.acc.x = s.acc.x * s1 + x2 * s2;
    s.acc.y = s.acc.y * s1 + y2 * s2;
    s.acc.z = s.acc.z * s1 + z2 * s2;
    s.acc.w = s.acc.w * s1 + u2 * s2;
    s.m = M;
}

__device__ __forceinline__ int merge_d0() { return 32 * (int)(threadIdx.x >> 6) + 4 * (int)((threadIdx.x & 63) >> 3); }

// The sources of a row are list A then list B, as one list of A.n + B.n: source k is A's k-th
// for k < A.n, else B's (k - A.n)-th. Lane r of each 8-lane group takes sources k0 + r + 8 u
// (u < kMergeU), loaded unconditionally: a lane past the last source reloads the last one, and
// the list a source comes from is a per-lane select of its address, so every lane issues the same
// loads and no load waits for another (conditional loads would make the compiler copy the
// results, and wait for them, where the branches join). 8 kMergeU sources per round trip.
__device__ __forceinline__ void merge_load(const MSrc& A, const MSrc& B, int k0, float (&l)[kMergeU],
                                           float4 (&o)[kMergeU]) {
    const int r = threadIdx.x & 7, d0 = merge_d0(), n = A.n + B.n;
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
        const int k = min(k0 + r + 8 * u, n - 1);
        const bool inA = k < A.n;
        const size_t i = inA ? (size_t)k * A.stride : (size_t)(k - A.n) * B.stride;
        const float* lp = inA ? A.lse : B.lse;
        const float* op = inA ? A.o : B.o;
        l[u] = lp[i];
        o[u] = *reinterpret_cast<const float4*>(op + i * kHeadDim + d0);
    }
}
// Folds this lane's loaded sources into s in order, branch-free (a dropped or empty source weighs 0
// and its values are replaced, not multiplied, so unused slots may hold anything): with every
// loaded value used unconditionally, the compiler keeps all the loads ahead of the first wait.
// For a kept source this is the online log-sum-exp rule: the running state (m, ws, acc) is rescaled
// by exp(m - max(m, l)) (exactly 1 when l <= m) and the source (lse l, normalized output o) added
// with weight exp(l - max(m, l)); an empty source (l = -inf) weighs 0. keepA(k) drops sources of
// list A (B's are all kept).
template <class KeepA>
__device__ __forceinline__ void merge_fold(MState& s, const MSrc& A, const MSrc& B, int k0,
                                           const float (&l)[kMergeU], const float4 (&o)[kMergeU],
                                           KeepA keepA) {
    const int r = threadIdx.x & 7, n = A.n + B.n;
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
        const int k = k0 + r + 8 * u;
        const bool ok = k < n && (k >= A.n || keepA(k)) && l[u] != -INFINITY;
        const float lv = ok ? l[u] : -INFINITY;
        const float4 ov = ok ? o[u] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float mn = fmaxf(s.m, lv);
        const float sc = (s.m == -INFINITY) ? 0.f : fast_exp2((s.m - mn) * kLog2e);
        const float w = ok ? fast_exp2((lv - mn) * kLog2e) : 0.f;
        s.ws = fmaf(s.ws, sc, w);
        s.acc.x = fmaf(w, ov.x, s.acc.x * sc);
        s.acc.y = fmaf(w, ov.y, s.acc.y * sc);
        s.acc.z = fmaf(w, ov.z, s.acc.z * sc);
        s.acc.w = fmaf(w, ov.w, s.acc.w * sc);
        s.m = mn;
    }
}

template <class KeepA>
__device__ __forceinline__ MState merge_lanes(const MSrc& A, const MSrc& B, KeepA keepA) {
    constexpr int SPT = 8 * kMergeU;   // sources per round trip
    MState s{-INFINITY, 0.f, make_float4(0.f, 0.f, 0.f, 0.f)};
    const int n = A.n + B.n;
    if (n > 0) {
        float l[kMergeU];
        float4 o[kMergeU];
        merge_load(A, B, 0, l, o);
        __builtin_amdgcn_sched_barrier(0);   // every load above is issued before anything waits
        merge_fold(s, A, B, 0, l, o, keepA);
        for (int k0 = SPT; k0 < n; k0 += SPT) {
            merge_load(A, B, k0, l, o);
            merge_fold(s, A, B, k0, l, o, keepA);
        }
    }
    mstate_fold_dpp<0xB1>(s);    // quad_perm [1,0,3,2]
    mstate_fold_dpp<0x4E>(s);    // quad_perm [2,3,0,1]
    mstate_fold_dpp<0x141>(s);   // row_half_mirror: the other quad of the 8-lane half row
    return s;
}

// Writes a merged row: lane 0 of each 8-lane group its 4 fp16 outputs, the first of them the lse.
// A row whose every source is empty gets out = 0, lse = -inf.
__device__ __forceinline__ void merge_store(const MState& s, _Float16* out_row, float* lse_out) {
    if ((threadIdx.x & 7) != 0) return;
    const int d0 = merge_d0();
    const float inv = s.ws > 0.f ? 1.f / s.ws : 0.f;
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 hv = {(_Float16)(s.acc.x * inv), (_Float16)(s.acc.y * inv), (_Float16)(s.acc.z * inv),
                   (_Float16)(s.acc.w * inv)};
    *reinterpret_cast<h4*>(out_row + d0) = hv;
    if (d0 == 0) *lse_out = s.ws > 0.f ? s.m + fast_log2(s.ws) * kLn2 : -INFINITY;
}

// ---- uniform chunks: the reference's decode_partial launch shape -------------------------
template <class C>
__global__ __launch_bounds__(C::NT) void decode_partial_kernel(PartialArgs a) {
    constexpr int G = C::G;
    __shared__ Smem<G, C::NW> sm;
    const int chunk = blockIdx.x;
    const int b = blockIdx.y / a.Hkv, kvh = blockIdx.y % a.Hkv;
    const int pb = a.kv_indptr[b];
    const int np = a.kv_indptr[b + 1] - pb;
    const int len = np > 0 ? (np - 1) * kPage + min(kPage, max(1, a.kv_last[b])) : 0;
    const int kbeg = a.kv_start + chunk * a.chunk_tokens;
    const int kend = min(len, kbeg + a.chunk_tokens);
    process_range<C>(sm, a.q + ((size_t)b * a.Hq + kvh * G) * kHeadDim, a.k, a.v,
                     a.kv_indices + pb, 0, kbeg, kend, a.Hkv, kvh, a.scale_log2);
    if (a.out != nullptr) {
        // the only chunk: its normalized state is the result (the merge's weight would be 1)
        const size_t row0 = (size_t)b * a.Hq + kvh * G;
        for (int idx = threadIdx.x; idx < G * kHeadDim; idx += C::NT) {
            const int h = idx / kHeadDim, d = idx % kHeadDim;
            a.out[(row0 + h) * kHeadDim + d] = (_Float16)sm.fo[h][d];
            if (d == 0) a.lse[row0 + h] = sm.flse[h];
        }
        return;
    }
    for (int idx = threadIdx.x; idx < G * kHeadDim; idx += C::NT) {
        const int h = idx / kHeadDim, d = idx % kHeadDim;
        const size_t slot = ((size_t)b * a.Hq + kvh * G + h) * a.part_stride + a.chunk_base + chunk;
        a.part_o[slot * kHeadDim + d] = sm.fo[h][d];
        if (d == 0) a.part_lse[slot] = sm.flse[h];
    }
}

// ---- log-sum-exp merge: the reference's merge_states launch shape -------------------------
// One workgroup per row, `num_chunks` consecutive partial slots.
__global__ __launch_bounds__(kMergeThreads) void merge_states_kernel(const float* __restrict__ part_o,
                                                                      const float* __restrict__ part_lse,
                                                                      _Float16* __restrict__ out,
                                                                      float* __restrict__ lse_out,
                                                                      int num_chunks) {
    const size_t row = blockIdx.x;
    const MSrc A{part_lse + row * num_chunks, part_o + row * num_chunks * kHeadDim, 1, num_chunks};
    const MSrc B{part_lse, part_o, 1, 0};
    const MState st = merge_lanes(A, B, [](int) { return true; });
    merge_store(st, out + row * kHeadDim, lse_out + row);
}

// ---- balanced launch -------------------------------------------------------------------------
// Merge of the pairs listed by the planner: one workgroup per row (entry, head). Sources: the
// pair's partial slots in order, then the row's extra partials (cascade prefix chunks). A list
// whose header does not carry the launch's tag, or an entry outside the batch or the workspace's
// slots, is someone else's bytes: the row is left alone.
// RECT (slots laid out by entry, cmax > 0): the list header, the entry and every partial are loaded
// in one round trip (the header and entry as vector loads through a zero lane offset the compiler
// cannot see through, so that they count against the same counter as the partials and nothing is
// waited for before all are issued). Otherwise the partials follow the entry.
template <bool RECT>
__global__ __launch_bounds__(kMergeThreads) void merge_split_kernel(MergeArgs a) {
    const int G = a.G, e = blockIdx.x / G, h = blockIdx.x - e * G;
    int z = 0;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    // header {tag, n_entries, cmax, 0} and entry {b, kvh, slot0, nc}
    const int4 hd = *reinterpret_cast<const int4*>(a.list + z);
    const int4 en = *reinterpret_cast<const int4*>(a.list + 4 + 4 * (size_t)e + z);
    const int n_extra = a.n_extra;
    MState st;
    if constexpr (RECT) {
        const int cmax = a.cmax;
        const size_t sl0 = (size_t)e * cmax * G + h;   // slot e * cmax, head h
        const size_t row = (size_t)e * G + h;          // with extra partials entry e is pair e
        const MSrc A{a.part_lse + sl0, a.part_o + sl0 * kHeadDim, (size_t)G, cmax};
        const MSrc B{a.extra_lse + row * n_extra, a.extra_o + row * n_extra * kHeadDim, 1, n_extra};
        st = merge_lanes(A, B, [&](int k) { return k < en.w; });
        if (en.w > cmax || (n_extra > 0 && (int64_t)en.x * a.Hkv + en.y != (int64_t)e)) return;
    } else {
        if (hd.x != a.tag || en.z < 0 || en.w < 0 || (int64_t)en.z + en.w > a.n_slots) return;
        if (en.x < 0 || en.x >= a.B || en.y < 0 || en.y >= a.Hkv) return;
        const size_t sl0 = (size_t)en.z * G + h;
        const size_t row = ((size_t)en.x * a.Hkv + en.y) * G + h;
        const MSrc A{a.part_lse + sl0, a.part_o + sl0 * kHeadDim, (size_t)G, en.w};
        const MSrc B{a.extra_lse + row * n_extra, a.extra_o + row * n_extra * kHeadDim, 1, n_extra};
        st = merge_lanes(A, B, [](int) { return true; });
    }
    if (hd.x != a.tag || en.x < 0 || en.x >= a.B || en.y < 0 || en.y >= a.Hkv) return;
    const size_t orow = ((size_t)en.x * a.Hkv + en.y) * G + h;
    merge_store(st, a.out + orow * kHeadDim, a.lse + orow);
}

// Per-segment merge scratch of the balanced kernel: the raw online-softmax state of every row
// group of every wave (NS = waves x row groups sources), then per-source weights. o rows are
// padded by 4 floats so that the row groups of a wave, which write the same columns, fall in
// different LDS banks. The o rows hold HP of the G heads at a time (the flush takes G / HP passes).
template <int G, int NS, int HP = G>
struct BalSmem {
    static constexpr int OP = kHeadDim + 4;
    float m[NS][G];
    float l[NS][G];
    float o[NS][HP][OP];
    float alpha[G][NS];       // exp(m_src - M) per head and source
    float rinv[G];            // 1 / L
    float lse[G];
};

template <class C>
__device__ __forceinline__ void reset_state(WaveState<C>& st) {
#pragma unroll
    for (int h = 0; h < C::G; ++h) {
        st.m[h] = -INFINITY;
        st.l[h] = 0.f;
#pragma unroll
        for (int d = 0; d < C::DPL; ++d) st.o[h][d] = 0.f;
    }
}

// Reduction (max or sum) over the lanes that agree modulo G (G in 1, 2, 4, 8), leaving the result
// in every one of them, in the VALU: quad permutations for lane distances 1 and 2, row
// rotations by 8 and 4 within a 16-lane row (after which every lane of the row holds the result
// of its class), and the row-pair swaps across rows.
template <int G, bool MAX>
__device__ __forceinline__ float class_reduce(float v) {
    auto op = [](float x, float y) { return MAX ? fmaxf(x, y) : x + y; };
    if constexpr (G == 1) v = op(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
    if constexpr (G <= 2) v = op(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
    v = op(v, dpp<0x128>(v));                        // row_ror:8
    if constexpr (G <= 4) v = op(v, dpp<0x124>(v));  // row_ror:4
    float x, y;
    row_pair<false>(v, x, y);
    row_pair<true>(op(x, y), x, y);
    return op(x, y);
}

// End of a segment. Every row group of every wave is one source state (max, sum, output slice);
// all of them go to LDS unmerged, one wave turns the per-source maxima into weights, and each
// thread forms four outputs as one weighted sum over the sources, in source order. Writes the G
// rows as the final fp16 out / lse (slot < 0) or as partial slot `slot` (normalized o, lse). The
// raw outputs go through LDS HP heads at a time (HP = G: one pass).
template <class C, int HP>
__device__ __forceinline__ void flush_segment(BalSmem<C::G, C::NW * C::RPI, HP>& sm, WaveState<C>& st,
                                              KArgPtr a, size_t row0, int slot,
                                              int tid = threadIdx.x) {
    constexpr int G = C::G, LPR = C::LPR, NS = C::NW * C::RPI;
    // one wave computes the source weights: lane = s * G + h covers sources s + j * SL, j < J
    constexpr int SL = 64 / G, J = (NS + SL - 1) / SL;
    static_assert(NS % 4 == 0 && HP * 32 <= C::NT && G % HP == 0, "float4 passes");
    // (tid: the thread's index among the C::NT threads that flush this state; every thread of the
    // workgroup calls it, as it holds barriers)
    const int lane = tid & 63, c = lane % LPR;
    const int src = (tid >> 6) * C::RPI + lane / LPR;
#pragma unroll
    for (int hp = 0; hp < G / HP; ++hp) {
#pragma unroll
        for (int hh = 0; hh < HP; ++hh)
#pragma unroll
            for (int kk = 0; kk < C::PPL; ++kk) {
                const int h = hp * HP + hh;
                float4* dst = reinterpret_cast<float4*>(&sm.o[src][hh][(kk * LPR + c) * 8]);
                dst[0] = make_float4(st.o[h][kk * 8 + 0], st.o[h][kk * 8 + 1], st.o[h][kk * 8 + 2], st.o[h][kk * 8 + 3]);
                dst[1] = make_float4(st.o[h][kk * 8 + 4], st.o[h][kk * 8 + 5], st.o[h][kk * 8 + 6], st.o[h][kk * 8 + 7]);
            }
        if (hp == 0 && c == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                sm.m[src][h] = st.m[h];
                sm.l[src][h] = st.l[h];
            }
        }
        __syncthreads();
        if (hp == 0) {
            if (tid < 64) {
                const int s0 = tid / G, h = tid % G;
                float mv[J];
                float M = -INFINITY;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const int s = s0 + j * SL;
                    mv[j] = s < NS ? sm.m[s][h] : -INFINITY;
                    M = fmaxf(M, mv[j]);
                }
                M = class_reduce<G, true>(M);
                float L = 0.f;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const int s = s0 + j * SL;
                    const float al = (mv[j] == -INFINITY) ? 0.f : fast_exp2(mv[j] - M);
                    if (s < NS) {
                        sm.alpha[h][s] = al;
                        L = fmaf(al, sm.l[s][h], L);
                    }
                }
                L = class_reduce<G, false>(L);
                if (tid < G) {
                    sm.rinv[h] = L > 0.f ? 1.f / L : 0.f;
                    sm.lse[h] = L > 0.f ? (M + fast_log2(L)) * kLn2 : -INFINITY;
                }
            }
            __syncthreads();
        }
        if (tid < HP * 32) {
            const int hh = tid / 32, h = hp * HP + hh, d0 = 4 * (tid % 32);
            float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int s4 = 0; s4 < NS; s4 += 4) {
                const float4 al = *reinterpret_cast<const float4*>(&sm.alpha[h][s4]);
                const float alv[4] = {al.x, al.y, al.z, al.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float4 ov = *reinterpret_cast<const float4*>(&sm.o[s4 + u][hh][d0]);
                    O.x = fmaf(alv[u], ov.x, O.x);
                    O.y = fmaf(alv[u], ov.y, O.y);
                    O.z = fmaf(alv[u], ov.z, O.z);
                    O.w = fmaf(alv[u], ov.w, O.w);
                }
            }
            const float ri = sm.rinv[h];
            O.x *= ri;
            O.y *= ri;
            O.z *= ri;
            O.w *= ri;
            if (slot < 0) {
                typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                const h4 hv = {(_Float16)O.x, (_Float16)O.y, (_Float16)O.z, (_Float16)O.w};
                *reinterpret_cast<h4*>(a->out + (row0 + h) * kHeadDim + d0) = hv;
                if (d0 == 0) a->lse[row0 + h] = sm.lse[h];
            } else {
                const int ps = a->part_stride;
                const size_t e = ps > 0 ? (row0 + h) * (size_t)ps + slot : (size_t)slot * G + h;
                *reinterpret_cast<float4*>(a->part_o + e * kHeadDim + d0) = O;
                if (d0 == 0) a->part_lse[e] = sm.lse[h];
            }
        }
        __syncthreads();   // sm is reused by the next pass or segment
    }
}

// One workgroup of 4 waves (one per SIMD) per CU walks its list of segments. Wave i takes pages
// i, i+4, ... of each segment; its pages of all segments form one stream, each segment's share
// padded to a multiple of the ring depth NBUF so that a page's ring slot is fixed at compile
// time. The ring runs across segment boundaries: the next segment's first pages are in flight
// while a segment is flushed. Partials are written with plain stores and merged by a second
// kernel, so no workgroup waits for another.
// COMPACT (the fused cascade step at G = 8, so that a CU holds it beside a prefix workgroup):
// the flush passes 4 heads at a time, and q rows are staged for at most kStepSegMax segments (the
// planner caps such a plan's segments per workgroup).
template <class C, bool COMPACT = false>
struct BalShared {
    static constexpr int HP = COMPACT && C::G > 4 ? 4 : C::G;        // heads per flush pass
    static constexpr int SEGS = COMPACT ? kStepSegMax : kSegMax;      // segments with staged q rows
    BalSmem<C::G, C::NW * C::RPI, HP> sm;
    int pg[kRangeMax];                             // the workgroup's page ids
    u32x4 qs[SEGS][C::G * kHeadDim / 8];           // q rows of each segment
    int sd[kBalDescInts];                          // descriptor block: header, then segments
};

// The segments staged in S.sd (nseg of them, at most S's SEGS; page ids of a page-range plan
// already in S.pg): their q rows and, for other plans, their page ids (positions from the
// descriptors, in kv_indices of the argument block) are loaded in one round trip, then every
// wave streams its pages of all segments through one ring, flushing each segment at its end.
// All threads of the workgroup call it.
template <class C, bool COMPACT, bool RANGES>
__device__ __forceinline__ void run_segments(const BalArgs& a, BalShared<C, COMPACT>& S, int nseg,
                                             bool qpre = false) {
    constexpr int G = C::G, NW = C::NW, NT = C::NT, NBUF = C::NBUF, LPR = C::LPR;
    auto& sm = S.sm;
    int* pg = S.pg;
    auto& qs = S.qs;
    int* sd = S.sd;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane / LPR, c = lane % LPR;
    int* seg = sd + 8;
    auto fld = [&](int si, int f) { return __builtin_amdgcn_readfirstlane(seg[si * kSegInts + f]); };
    constexpr int PMAX = kRangeMax / NT, QPS = G * kHeadDim / 8;
    constexpr int QMAX = (BalShared<C, COMPACT>::SEGS * QPS + NT - 1) / NT;
    const uint32_t page_bytes = (uint32_t)(kPage * a.Hkv * 256);
    const uint32_t lbase = (uint32_t)(r * a.Hkv * 256 + c * 16);
    const uint32_t rstride = (uint32_t)(C::RPI * a.Hkv * 256);
    auto wcount = [&](int npg) { return npg > wave ? (npg - wave + NW - 1) / NW : 0; };

    // prefetch cursor: segment ps, slot pslot of this wave's (padded) share pcnt / ppad
    int ps = 0, pslot = 0, pcnt = 0, ppad = 0;
    auto seek = [&]() {
        while (ps < nseg) {
            pcnt = wcount(fld(ps, 3));
            ppad = (pcnt + NBUF - 1) / NBUF * NBUF;
            if (ppad > 0) break;
            ++ps;
        }
    };
    auto issue = [&](PageRegs<C>& buf) {
        const uint8_t* kb = kargs()->k;
        const uint8_t* vb = kargs()->v;
        uint32_t nrec = 0;
        if (ps < nseg && pslot < pcnt) {
            const int kvh = fld(ps, 1);
            const int pid = __builtin_amdgcn_readfirstlane(pg[fld(ps, 2) + wave + NW * pslot]);
            const size_t off = (size_t)(uint32_t)pid * page_bytes + (size_t)kvh * 256;
            kb += off;
            vb += off;
            nrec = page_bytes - (uint32_t)kvh * 256;
        }
        load_page_rsrc<C>(buf, page_rsrc(kb, nrec), page_rsrc(vb, nrec), lbase, rstride);
        if (ps < nseg && ++pslot == ppad) {
            ++ps;
            pslot = 0;
            seek();
        }
    };

    // round trip 2: the q rows of every segment, the page ids of the other plans (item i of the
    // workgroup's page list is found in the segment whose range [qa, qa + npg) holds it), and for
    // a page-range plan the first pages of the ring, all issued before any is waited for
    PageRegs<C> buf[NBUF];
    {
        const int npages = fld(nseg - 1, 2) + fld(nseg - 1, 3);
        const _Float16* qp = kargs()->q;
        const int32_t* kvi = kargs()->kv_indices;
        // page-table positions of the page list first (LDS reads only: a search loop with loads
        // in flight would make the compiler wait for them at every iteration)
        int src[PMAX];
        if constexpr (!RANGES) {
#pragma unroll
            for (int k = 0; k < PMAX; ++k) {
                const int i = tid + k * NT;
                src[k] = -1;
                if (i < npages) {
                    int si = 0;
                    while (si + 1 < nseg && seg[(si + 1) * kSegInts + 2] <= i) ++si;
                    src[k] = seg[si * kSegInts + 6] + (i - seg[si * kSegInts + 2]);
                }
            }
        }
        // (every load is issued, past the last segment from segment 0's rows, so that the number
        // of loads in flight is the same on every path and the waits below stay exact)
        u32x4 qv4[QMAX];
        if (!qpre) {
#pragma unroll
            for (int k = 0; k < QMAX; ++k) {
                const int j = tid + k * NT < nseg * QPS ? tid + k * NT : 0;
                const int si = j / QPS;
                const size_t row = (size_t)seg[si * kSegInts] * a.Hq + (size_t)seg[si * kSegInts + 1] * G;
                qv4[k] = reinterpret_cast<const u32x4*>(qp + row * kHeadDim)[j % QPS];
            }
        }
        int pv[PMAX];
        if constexpr (!RANGES) {
            // (unconditional within the list, so one round trip; none at all for a workgroup whose
            // items hold no page, whose kv_indices may be empty)
            if (npages > 0) {
#pragma unroll
                for (int k = 0; k < PMAX; ++k) pv[k] = kvi[max(src[k], 0)];
            }
        } else {
            seek();
#pragma unroll
            for (int u = 0; u < NBUF - 1; ++u) issue(buf[u]);
        }
        // keeps the stores below after the loads above: the q rows are waited for while the
        // first pages are still in flight
        asm volatile("" ::: "memory");
        if (!qpre) {
#pragma unroll
            for (int k = 0; k < QMAX; ++k)
                if (tid + k * NT < nseg * QPS) qs[(tid + k * NT) / QPS][(tid + k * NT) % QPS] = qv4[k];
        }
        if constexpr (!RANGES) {
#pragma unroll
            for (int k = 0; k < PMAX; ++k)
                if (tid + k * NT < npages) pg[tid + k * NT] = pv[k];
        }
    }
    __syncthreads();
    PD_STAMP(2);
    if constexpr (!RANGES) {
        seek();
#pragma unroll
        for (int u = 0; u < NBUF - 1; ++u) issue(buf[u]);
    }

    WaveState<C> st;
    reset_state<C>(st);
    for (int si = 0; si < nseg; ++si) {
        const int npg = fld(si, 3), t0 = fld(si, 4), t1 = fld(si, 5);
        const int tbase = t0 & ~(kPage - 1);   // first token of the segment's first page
        f16x2 qv[G][C::PPL][4];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int kk = 0; kk < C::PPL; ++kk) {
                const u32x4 raw = qs[qpre ? 0 : si][h * (kHeadDim / 8) + kk * LPR + c];
#pragma unroll
                for (int e = 0; e < 4; ++e) qv[h][kk][e] = as_h2(raw[e]);
            }
        const int cnt = wcount(npg);
        for (int blk = 0; blk < cnt; blk += NBUF) {
#pragma unroll
            for (int u = 0; u < NBUF; ++u) {
                issue(buf[(u + NBUF - 1) % NBUF]);
                if (blk + u < cnt)
                    page_step<C>(st, buf[u], qv, tbase + (wave + NW * (blk + u)) * kPage, r, t0, t1,
                                 a.scale_log2);
            }
            if (si == 0 && blk == 0) PD_STAMP(3);
        }
        if (si < 12) PD_STAMP(4 + 2 * si);
        flush_segment<C, BalShared<C, COMPACT>::HP>(sm, st, kargs(),
                                                    (size_t)fld(si, 0) * a.Hq + (size_t)fld(si, 1) * G,
                                                    fld(si, 7));
        reset_state<C>(st);
        if (si < 12) PD_STAMP(5 + 2 * si);
    }
    PD_STAMP(31);
}


// ---- the paired decode: two kv heads per workgroup, pages staged in LDS --------------------
// A 4-wave workgroup runs two workgroups of a page-range plan, w = 2 x and 2 x + 1: kv heads
// 2k and 2k + 1 over the same pages. Waves 0-1 serve the first head and waves 2-3 the second,
// each pair of waves as a plan workgroup of two waves (C::NW = 2), wave i of a head taking pages
// i, i + 2, ... of every segment. Reading the two heads' rows of a page together (1 KB of every
// 2 KB token row at once) streams faster than one head's 256-byte rows. The page ring goes
// through LDS instead of VGPRs: each wave moves its pages with 16-byte buffer loads straight
// into its own LDS slots (buffer_load ... lds; lane l's pieces land at 16 l of each 1 KB, and
// lane l reads the same bytes back), two slots per wave. The compiler makes a workgroup barrier
// wait for every LDS-bound load in flight, so no barrier is placed while pages are in flight
// except the flushes': q rows go straight to registers (each lane its own pieces), one segment
// ahead, instead of through LDS.
template <class C>
struct PairShared {
    static constexpr int SLOT = C::RG * C::PPL * 1024 * 2;   // one page of one head: K then V
    BalSmem<C::G, C::NW * C::RPI> sm[2];           // flush scratch of each head's waves
    int sd[2][kBalDescInts];                       // the two heads' descriptor blocks
    int pg[kRangeMax];                             // the range's page ids (the same for both heads)
    __attribute__((aligned(16))) uint8_t ring[2 * C::NW][2][SLOT];
};

typedef __attribute__((address_space(3))) void lds_void;

// One page of one head into a wave's LDS slot: lane l's pieces of row group i at
// slot + (i PPL + kk) * 1024 + 16 l, K then V. Same offsets, resources and cache policy as the
// VGPR ring's loads (a padding slot's zero-size resources make no memory access).
template <class C>
__device__ __forceinline__ void dma_page(uint8_t* slot, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                         uint32_t lbase, uint32_t rstride) {
    constexpr int HALF = C::RG * C::PPL * 1024;
#pragma unroll
    for (int i = 0; i < C::RG; ++i)
#pragma unroll
        for (int kk = 0; kk < C::PPL; ++kk) {
            const int off = (int)(lbase + i * rstride + kk * (C::LPR * 16));
            uint8_t* d = slot + (i * C::PPL + kk) * 1024;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)d, 16, off, 0, 0, 2);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(d + HALF), 16, off, 0, 0, 2);
        }
}
template <class C>
__device__ __forceinline__ void lds_page(PageRegs<C>& pr, const uint8_t* slot, int lane) {
    constexpr int HALF = C::RG * C::PPL * 1024;
#pragma unroll
    for (int i = 0; i < C::RG; ++i)
#pragma unroll
        for (int kk = 0; kk < C::PPL; ++kk) {
            const uint8_t* d = slot + (i * C::PPL + kk) * 1024 + 16 * lane;
            pr.k[i][kk] = *reinterpret_cast<const u32x4*>(d);
            pr.v[i][kk] = *reinterpret_cast<const u32x4*>(d + HALF);
        }
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt at their maximum: no wait on them).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14));
}
// s_waitcnt lgkmcnt(0) alone.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Workgroup x of the paired decode (page-range plans only; the plan's Hkv is even). Both heads'
// descriptor blocks are staged; everything that decides the control flow (segments, pages,
// tokens) is read from the first, so both halves reach every barrier together. The second head's
// block contributes its partial slots.
template <class C>
__device__ __forceinline__ void pair_body(const BalArgs& a, PairShared<C>& P, int x) {
    constexpr int G = C::G, NW = C::NW, NT2 = 2 * C::NT, LPR = C::LPR, PPL = C::PPL;
    constexpr int PMAX = kRangeMax / NT2;
    constexpr int DPER = (2 * kBalDescInts + NT2 - 1) / NT2;
    constexpr int OPS = 2 * C::RG * C::PPL;       // buffer loads per page
    static_assert(C::NBUF == 2, "two LDS slots and two register sets per wave");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = wave / NW, lw = wave % NW, ltid = tid - half * C::NT;
    const int r = lane / LPR, c = lane % LPR;
    int* sd0 = P.sd[0];
    int* seg0 = sd0 + 8;
    auto fld = [&](int si, int f) { return __builtin_amdgcn_readfirstlane(seg0[si * kSegInts + f]); };
    PD_STAMP(0);
    // round trip 1: both descriptor blocks and the range's page ids
    const int w0 = 2 * x;
    const int64_t g = w0 / a.Hkv, nnz = kargs()->nnz, ng = kargs()->ngroups;
    const int64_t lo = nnz * g / ng, hi = nnz * (g + 1) / ng;
    {
        const int32_t* desc = kargs()->desc + (size_t)w0 * kBalDescInts;
        const int32_t* kvi = kargs()->kv_indices + lo;
        int dv[DPER], pv[PMAX];
#pragma unroll
        for (int k = 0; k < DPER; ++k) {
            const int i = tid + k * NT2;
            dv[k] = i < 2 * kBalDescInts ? desc[i] : 0;
        }
        const int npr = (int)(hi - lo);
#pragma unroll
        for (int k = 0; k < PMAX; ++k) {
            const int i = tid + k * NT2;
            pv[k] = i < npr ? kvi[i] : 0;
        }
#pragma unroll
        for (int k = 0; k < DPER; ++k) {
            const int i = tid + k * NT2;
            if (i < 2 * kBalDescInts) P.sd[i / kBalDescInts][i % kBalDescInts] = dv[k];
        }
#pragma unroll
        for (int k = 0; k < PMAX; ++k)
            if (tid + k * NT2 < npr) P.pg[tid + k * NT2] = pv[k];
    }
    __syncthreads();
    PD_STAMP(1);
    // (uniform: every thread leaves) either block foreign or empty, or the blocks disagree
    const int nseg = __builtin_amdgcn_readfirstlane(sd0[0]);
    const int kvh0 = __builtin_amdgcn_readfirstlane(nseg > 0 ? seg0[1] : 0);
    if (nseg <= 0 || nseg > kSegMax || nseg != __builtin_amdgcn_readfirstlane(P.sd[1][0]) ||
        __builtin_amdgcn_readfirstlane(sd0[1]) != kargs()->tag ||
        __builtin_amdgcn_readfirstlane(P.sd[1][1]) != kargs()->tag || kvh0 < 0 || kvh0 + 1 >= a.Hkv)
        return;
    const int kvh = kvh0 + half;

    const uint32_t page_bytes = (uint32_t)(kPage * a.Hkv * 256);
    const uint32_t lbase = (uint32_t)(r * a.Hkv * 256 + c * 16);
    const uint32_t rstride = (uint32_t)(C::RPI * a.Hkv * 256);
    auto wcount = [&](int npg) { return npg > lw ? (npg - lw + NW - 1) / NW : 0; };
    int ps = 0, pslot = 0, pcnt = 0, ppad = 0;
    auto seek = [&]() {
        while (ps < nseg) {
            pcnt = wcount(fld(ps, 3));
            ppad = (pcnt + 1) / 2 * 2;
            if (ppad > 0) break;
            ++ps;
        }
    };
    // stream page k of this wave (padding included) goes to LDS slot k % 2 and register set k % 2
    int nissued = 0;
    auto issue = [&]() {
        const uint8_t* kb = kargs()->k;
        const uint8_t* vb = kargs()->v;
        uint32_t nrec = 0;
        if (ps < nseg && pslot < pcnt) {
            const int pid = __builtin_amdgcn_readfirstlane(P.pg[fld(ps, 2) + lw + NW * pslot]);
            const size_t off = (size_t)(uint32_t)pid * page_bytes + (size_t)kvh * 256;
            kb += off;
            vb += off;
            nrec = page_bytes - (uint32_t)kvh * 256;
        }
        dma_page<C>(P.ring[wave][nissued & 1], page_rsrc(kb, nrec), page_rsrc(vb, nrec), lbase, rstride);
        ++nissued;
        if (ps < nseg && ++pslot == ppad) {
            ++ps;
            pslot = 0;
            seek();
        }
    };
    // this lane's q pieces of segment si (head h, piece kk: dims (kk LPR + c) 8 .. + 7)
    auto qload = [&](int si, u32x4 (&q)[G][PPL]) {
        const _Float16* qp = kargs()->q + ((size_t)fld(si, 0) * a.Hq + (size_t)kvh * G) * kHeadDim;
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int kk = 0; kk < PPL; ++kk)
                q[h][kk] = *reinterpret_cast<const u32x4*>(qp + h * kHeadDim + (kk * LPR + c) * 8);
    };

    // round trip 2: the first segment's q pieces, then the first two pages of the ring
    u32x4 qn[G][PPL];
    qload(0, qn);
    seek();
    issue();
    issue();
    wait_vm<OPS>();            // page 0 (page 1 in flight)
    PageRegs<C> pr[2];
    lds_page<C>(pr[0], P.ring[wave][0], lane);
    PD_STAMP(2);

    WaveState<C> st;
    reset_state<C>(st);
    for (int si = 0; si < nseg; ++si) {
        const int npg = fld(si, 3), t0 = fld(si, 4), t1 = fld(si, 5);
        const int tbase = t0 & ~(kPage - 1);
        f16x2 qv[G][PPL][4];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int kk = 0; kk < PPL; ++kk)
#pragma unroll
                for (int e = 0; e < 4; ++e) qv[h][kk][e] = as_h2(qn[h][kk][e]);
        if (si + 1 < nseg) qload(si + 1, qn);   // (waited for at the next segment)
        const int cnt = wcount(npg);
        for (int blk = 0; blk < cnt; blk += 2) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                // page k (parity u) is in pr[u]; its slot is refilled with page k + 2 once the
                // reads of it are done; page k + 1 (in flight since the last step) is waited for
                // and read into pr[u ^ 1] while page k is computed
                wait_lgkm0();
                issue();
                wait_vm<OPS>();
                lds_page<C>(pr[u ^ 1], P.ring[wave][u ^ 1], lane);
                if (blk + u < cnt)
                    page_step<C>(st, pr[u], qv, tbase + (lw + NW * (blk + u)) * kPage, r, t0, t1,
                                 a.scale_log2);
            }
            if (si == 0 && blk == 0) PD_STAMP(3);
        }
        if (si < 12) PD_STAMP(4 + 2 * si);
        // this head's slot: its own block's field (the two blocks differ only in head and slot)
        const int slot = __builtin_amdgcn_readfirstlane(P.sd[half][8 + si * kSegInts + 7]);
        flush_segment<C, G>(P.sm[half], st, kargs(), (size_t)fld(si, 0) * a.Hq + (size_t)kvh * G, slot, ltid);
        reset_state<C>(st);
        if (si < 12) PD_STAMP(5 + 2 * si);
    }
    PD_STAMP(31);
}

// The body of one balanced-decode workgroup w (the kernel's argument block must start with the
// BalArgs `a`, which kargs() reads).
template <class C, bool UNI = false, bool COMPACT = false, bool RANGES = false>
__device__ __forceinline__ void balanced_body(const BalArgs& a, BalShared<C, COMPACT>& S, int w,
                                              const UniArgs* u = nullptr) {
    static_assert(!(UNI && RANGES), "the uniform split builds its own descriptors");
    constexpr int G = C::G, NT = C::NT;
    int* pg = S.pg;
    auto& qs = S.qs;
    int* sd = S.sd;
    const int tid = threadIdx.x;
    // Segment fields are staged in LDS (sd: a header of 8 ints, then the segments) and read back
    // wave-uniform by run_segments: global (vector) loads of them would count against the same
    // wait counter as the ring's page loads, and a non-uniform value in a buffer resource would
    // turn every page load into a loop over lanes.
    int* seg = sd + 8;
    // timestamps (timeline build only): 0 start, 1 descriptors (and page ids) staged, 2 q rows
    // staged, 3 the first ring step computed, 4 + 2 s / 5 + 2 s segment s streamed / flushed
    // (s < 12), 31 done; thread 0 of the workgroup
    PD_STAMP(0);
    constexpr int PMAX = kRangeMax / NT, QPS = G * kHeadDim / 8;
    // A page-range plan (RANGES: ngroups > 0) gives workgroup w = g * Hkv + kvh the pages
    // [lo, hi) of the page table (relative to kv_indptr[0]), lo = nnz g / ngroups: its page list is
    // known from the kernel arguments, so the page ids are loaded together with the descriptor
    // block, and the ring's first pages together with the q rows.
    int64_t lo = 0, hi = 0;
    bool qpre = false;   // q rows staged in round trip 1 (a one-sequence page-range plan)
    if constexpr (RANGES) {
        const int64_t g = w / a.Hkv, nnz = kargs()->nnz, ng = kargs()->ngroups;
        lo = nnz * g / ng;
        hi = nnz * (g + 1) / ng;
        qpre = kargs()->qrow_b >= 0;
    }
    int nseg;
    if constexpr (!UNI) {
        // round trip 1: the whole descriptor block (one int per thread), and the page ids of a
        // page-range plan
        const int32_t* desc = kargs()->desc + (size_t)w * kBalDescInts;
        const int32_t* kvi = kargs()->kv_indices + lo;   // (pointers read from the arguments once)
        const int dv = tid < kBalDescInts ? desc[tid] : 0;
        int pv[PMAX];
        const int npr = (int)(hi - lo);
#pragma unroll
        for (int k = 0; k < PMAX; ++k) {
            const int i = tid + k * NT;
            pv[k] = i < npr ? kvi[i] : 0;
        }
        // a one-sequence plan: the q rows of (qrow_b, this workgroup's kv head) in the same trip
        // (every segment uses them), so that round trip 2 carries only the ring's first pages
        u32x4 qv = {0u, 0u, 0u, 0u};
        if constexpr (RANGES) {
            if (qpre) {
                const size_t row = (size_t)kargs()->qrow_b * a.Hq + (size_t)(w % a.Hkv) * G;
                if (tid < QPS) qv = reinterpret_cast<const u32x4*>(kargs()->q + row * kHeadDim)[tid];
            }
        }
        if (tid < kBalDescInts) sd[tid] = dv;
#pragma unroll
        for (int k = 0; k < PMAX; ++k)
            if (tid + k * NT < npr) pg[tid + k * NT] = pv[k];
        if (qpre && tid < QPS) qs[0][tid] = qv;
        __syncthreads();
        PD_STAMP(1);
        nseg = __builtin_amdgcn_readfirstlane(sd[0]);
        // (uniform: every thread leaves) no segment, or not this plan's descriptor block: the
        // workspace was written over since the upload, and nothing here is to be trusted
        if (nseg <= 0 || nseg > BalShared<C, COMPACT>::SEGS ||
            __builtin_amdgcn_readfirstlane(sd[1]) != kargs()->tag)
            return;
    } else {
        // items w, w + W, ...: thread t builds the descriptor of the t-th (the decode_partial
        // rule, 01_decode_attention.cu:88-97: keys [kv_start + chunk * chunk_tokens, + chunk_tokens)
        // clipped to the sequence; an empty range writes 0 / -inf). t0 is the first key of the
        // range, which need not start a page: keys are numbered from its page's first token.
        nseg = min(u->per_wg, (u->n_items - w + a.W - 1) / a.W);
        if (nseg <= 0) return;   // uniform: the host sizes the grid so that every workgroup has items
        if (tid < nseg) {
            const int item = w + tid * a.W;
            const int pair = item / u->num_chunks, chunk = item - pair * u->num_chunks;
            const int b = pair / a.Hkv, kvh = pair - b * a.Hkv;
            const int pb = u->kv_indptr[b], np = u->kv_indptr[b + 1] - pb;
            // (a last-page length outside [1, 16] is clamped: no key past the sequence's pages)
            const int len = np > 0 ? (np - 1) * kPage + min(kPage, max(1, u->kv_last[b])) : 0;
            const int kbeg = u->kv_start + chunk * u->chunk_tokens;
            const int kend = max(kbeg, min(len, kbeg + u->chunk_tokens));
            const int pf = kbeg / kPage;
            int* sg = seg + tid * kSegInts;
            sg[0] = b;
            sg[1] = kvh;
            sg[3] = kend > kbeg ? (kend - 1) / kPage - pf + 1 : 0;
            sg[4] = kbeg;
            sg[5] = kend;
            sg[6] = pb + pf;
            sg[7] = a.out != nullptr ? -1 : u->chunk_base + chunk;
        }
        __syncthreads();
        // page-list offsets: exclusive prefix sum of the page counts
        if (tid < nseg) {
            int qa = 0;
            for (int j = 0; j < tid; ++j) qa += seg[j * kSegInts + 3];
            seg[tid * kSegInts + 2] = qa;
        }
        __syncthreads();
        PD_STAMP(1);
    }

    run_segments<C, COMPACT, RANGES>(a, S, nseg, qpre);
}

// ---- page ranges found on the device (the drop-in decode_attention without a host plan) -----
template <class C, bool COMPACT>
struct DevShared {
    BalShared<C, COMPACT> b;
    int ip[kDevMaxB + 1];      // kv_indptr
    int wx[2 * C::NW];         // per-wave piece counts and clip flags of the common-case guess
    int sc[C::NW + 1];         // block-scan scratch; sc[NW]: the current batch's first page
};

// Exclusive prefix sum of v over the workgroup's threads, in thread order, and the total. All
// threads call it (it holds two barriers).
template <int NW>
__device__ __forceinline__ int block_exscan(int v, int* sc, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) sc[wave] = x;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int t = sc[i];
        base += i < wave ? t : 0;
        tot += t;
    }
    __syncthreads();
    total = tot;
    return base + x - v;
}

// Workgroup w = g * Hkv + kvh: range g of the attended pages, kv head kvh. Thread t handles
// sequences 4 t .. 4 t + 3 (B <= kDevMaxB). One round trip loads kv_indptr and the last-page
// lengths. In the common case (keys from 0, no sequence cut short by the span) the attended pages
// of sequence b are all its pages, their prefix sums are kv_indptr[b] - kv_indptr[0], and a range's
// page ids are contiguous in kv_indices: that case is assumed at once, its page ids are loaded
// while one barrier settles whether it holds, and its pieces run as a host page-range plan's do.
// Otherwise two block scans give the prefix sums of the attended pages and the index of each
// sequence piece in the range, and the pieces run in batches of at most SEGS segments (a range of
// many short sequences), each batch like a host plan's workgroup (run_segments).
template <class C, bool COMPACT>
__device__ __forceinline__ void dev_body(const DevArgs& da, DevShared<C, COMPACT>& D, int w) {
    constexpr int G = C::G, NW = C::NW, NT = C::NT, SEGS = BalShared<C, COMPACT>::SEGS;
    constexpr int PMAX = kRangeMax / NT;
    static_assert(4 * NT >= kDevMaxB + 1, "four sequences per thread");
    const BalArgs& a = da.d;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, B = a.B, Hkv = a.Hkv;
    const int g = w / Hkv, kvh = w - g * Hkv;
    const int64_t NG = a.ngroups;
    PD_STAMP(0);
    // (unconditional loads at clamped indices, B >= 1: a conditional load per element would be
    // waited for before the next is issued)
    int ipv[4], lnv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int b = 4 * tid + k;
        ipv[k] = da.kv_indptr[min(b, B)];
        lnv[k] = da.kv_last[min(b, B - 1)];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (4 * tid + k <= B) D.ip[4 * tid + k] = ipv[k];
    __syncthreads();
    PD_STAMP(1);
    // (32-bit arithmetic from here on: page positions are int32, and a sequence's keys fit an int;
    // wave64 integer work costs four cycles an instruction, and 64-bit work twice that)
    const int ks = da.kv_start;   // >= 0
    const int ke = (int)min((int64_t)ks + da.span, (int64_t)INT_MAX);
    // The common-case guess (uniform: every thread takes the same branches on it). Its page ids
    // [ip0 + lo, ip0 + hi) lie in [ip0, kv_indptr[B]), entries of the page table whatever the
    // outcome; a range of more than kRangeMax pages (the guess being wrong) loads only the first.
    // They are loaded first, while the rest is worked out.
    const int ip0 = __builtin_amdgcn_readfirstlane(D.ip[0]);
    const int ipB = __builtin_amdgcn_readfirstlane(D.ip[B]);
    const bool guess = ks == 0 && ip0 >= 0 && ipB >= ip0;
    int N = guess ? ipB - ip0 : 0;
    int lo = (int)((int64_t)N * g / NG), hi = (int)((int64_t)N * (g + 1) / NG);
    // (branch-free loads at indices clamped into the range, or of kv_indptr[0] with no range to
    // load: the waits for the loads before them then count exactly, and none waits for these)
    int pv[PMAX];
    {
        const bool ok = guess && hi > lo;
        const int32_t* kvi = ok ? kargs()->kv_indices + ip0 + lo : da.kv_indptr;
        const int last = ok ? hi - lo - 1 : 0;
#pragma unroll
        for (int k = 0; k < PMAX; ++k) pv[k] = kvi[min(tid + k * NT, last)];
    }
    // attended pages of each sequence: keys [ks, min(len, ks + span)), from page ks / 16 (a
    // last-page length outside [1, 16] is clamped, as in the uniform split)
    const int ipn = D.ip[min(4 * tid + 4, B)];
    int cnt[4], lenv[4], pb[4], sum = 0, clipped = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int b = 4 * tid + k;
        const int np = b < B ? (k < 3 ? ipv[k + 1] : ipn) - ipv[k] : 0;
        const int len = np > 0 ? (np - 1) * kPage + min(kPage, max(1, lnv[k])) : 0;
        const int kend = min(len, ke);
        const int c = kend > ks ? (int)((uint32_t)(kend - 1) / kPage) - ks / kPage + 1 : 0;
        clipped |= c != np;
        cnt[k] = c;
        lenv[k] = len;
        pb[k] = b <= B ? ipv[k] - ip0 : N;
        sum += c;
    }
    // one barrier: the guess's per-wave piece counts and clip flags. Piece k of each thread is one
    // bit of a ballot, so the wave's exclusive prefix is four masked popcounts.
    int fl[4], nf = 0, x = 0, wn = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        fl[k] = cnt[k] > 0 && pb[k] < hi && pb[k] + cnt[k] > lo;
        nf += fl[k];
        const uint64_t m = __builtin_amdgcn_ballot_w64(fl[k] != 0);
        x += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
        wn += __builtin_popcountll(m);
    }
    const bool wclip = __builtin_amdgcn_ballot_w64(clipped != 0) != 0;
    if (lane == 0) {
        D.wx[wave] = wn;
        D.wx[NW + wave] = wclip;
    }
    __syncthreads();
    PD_STAMP(28);
    int f0 = x, ntot = 0, anyclip = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int t = D.wx[i];
        f0 += i < wave ? t : 0;
        ntot += t;
        anyclip |= D.wx[NW + i];
    }
    const bool fast = guess && !anyclip;
    if (!fast) {
        // prefix sums of the attended pages, then the pieces of the range
        int run = block_exscan<NW>(sum, D.sc, N);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            pb[k] = run;
            run += cnt[k];
        }
        lo = (int)((int64_t)N * g / NG);
        hi = (int)((int64_t)N * (g + 1) / NG);
        nf = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            fl[k] = cnt[k] > 0 && pb[k] < hi && pb[k] + cnt[k] > lo;
            nf += fl[k];
        }
        f0 = block_exscan<NW>(nf, D.sc, ntot);
    }
    if (w == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (4 * tid + k <= B) da.prefix[4 * tid + k] = pb[k];
    }
    if (lo == hi) {
        // an empty range (fewer pages than ranges): its slots are read as empty by the merge
        if (tid < 2 * G) a.part_lse[((size_t)2 * w + tid / G) * G + tid % G] = -INFINITY;
        return;
    }
    int* sd = D.b.sd;
    int* seg = sd + 8;
    // Descriptors of segments [sb, sb + nseg) whose page list starts at page bs0 of the attended
    // pages; the caller publishes them with a barrier.
    auto describe = [&](int sb, int nseg, int bs0) {
        int fi = f0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (!fl[k]) continue;
            const int si = fi++ - sb;
            if (si < 0 || si >= nseg) continue;
            const int b = 4 * tid + k;
            const int s0 = max(pb[k], lo), s1 = min(pb[k] + cnt[k], hi);
            const int pa0 = ks / kPage + (s0 - pb[k]), pa1 = ks / kPage + (s1 - pb[k]);
            const int kend = min(lenv[k], ke);
            int* sg = seg + si * kSegInts;
            sg[0] = b;
            sg[1] = kvh;
            sg[2] = s0 - bs0;
            sg[3] = s1 - s0;
            sg[4] = max(ks, pa0 * kPage);
            sg[5] = min(kend, pa1 * kPage);
            sg[6] = D.ip[b] + pa0;
            sg[7] = (s0 == pb[k] && s1 == pb[k] + cnt[k]) ? -1
                    : (s0 == lo && pb[k] < lo) ? 2 * w : 2 * w + 1;
        }
        if (tid == 0) sd[0] = nseg;
    };
    // The common case, every piece of the range in one batch: the range's page list is its pages,
    // and the segment runner is the last thing the workgroup does, so none of the state above stays
    // live through its page loop (which then compiles to the plan path's schedule: measured 7%
    // slower streaming otherwise).
    if (fast && ntot <= SEGS) {
        describe(0, ntot, lo);
#pragma unroll
        for (int k = 0; k < PMAX; ++k)
            if (tid + k * NT < hi - lo) D.b.pg[tid + k * NT] = pv[k];
        __syncthreads();
        PD_STAMP(30);
        run_segments<C, COMPACT, true>(a, D.b, ntot);
        return;
    }
    // Batches: each one's page list starts at its first segment's first page in the range.
    for (int sb = 0; sb < ntot; sb += SEGS) {
        const int nseg = min(SEGS, ntot - sb);
        {
            int fi = f0;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (fl[k]) {
                    if (fi == sb) D.sc[NW] = max(pb[k], lo);
                    ++fi;
                }
        }
        __syncthreads();
        const int bs0 = D.sc[NW];
        describe(sb, nseg, bs0);
        __syncthreads();
        run_segments<C, COMPACT, false>(a, D.b, nseg);
    }
}

// Merge of the sequences split over ranges: one workgroup per row (b, q head); the prefix sums
// written by the decode launch say which ranges hold sequence b's pages. A row of a sequence
// with no attended key gets 0 / -inf; a sequence within one range was written by its workgroup.
__global__ __launch_bounds__(kMergeThreads) void merge_ranges_kernel(DevMergeArgs a) {
    const int row = blockIdx.x, b = row / a.Hq, hq = row - b * a.Hq;
    const int kvh = hq / a.G, hh = hq - kvh * a.G;
    const int64_t pb = a.prefix[b], pe = a.prefix[b + 1], N = a.prefix[a.B];
    MState st{-INFINITY, 0.f, make_float4(0.f, 0.f, 0.f, 0.f)};
    if (pe > pb) {
        const int64_t NG = a.ngroups;
        const int64_t g0 = ((pb + 1) * NG - 1) / N, g1 = (pe * NG - 1) / N;
        if (g0 == g1) return;
        const size_t i0 = ((size_t)(g0 * a.Hkv + kvh) * 2 + 1) * a.G + hh;       // slot 2 w + 1 of g0
        const size_t i1 = ((size_t)((g0 + 1) * a.Hkv + kvh) * 2) * a.G + hh;     // slot 2 w of g0 + 1
        const MSrc A{a.part_lse + i0, a.part_o + i0 * kHeadDim, 1, 1};
        const MSrc Bs{a.part_lse + i1, a.part_o + i1 * kHeadDim, (size_t)2 * a.Hkv * a.G, (int)(g1 - g0)};
        st = merge_lanes(A, Bs, [](int) { return true; });
    } else {
        // (the fold leaves the empty state: out 0, lse -inf)
        const MSrc E{a.part_lse, a.part_o, 1, 0};
        st = merge_lanes(E, E, [](int) { return true; });
    }
    merge_store(st, a.out + (size_t)row * kHeadDim, a.lse + row);
}

// At G = 8 the per-page VALU work is about twice G = 4's and no longer hides under the page's
// memory time with one wave per SIMD, so the kernel uses the compact LDS layout (61 KB) and the
// planner gives it two workgroups per CU: the two waves on each SIMD overlap one's arithmetic with
// the other's loads.
template <class C, bool RANGES>
__global__ __launch_bounds__(C::NT) void decode_balanced_kernel(BalArgs a) {
    __shared__ BalShared<C, (C::G > 4)> S;
    balanced_body<C, false, (C::G > 4), RANGES>(a, S, blockIdx.x);
}

// The paired decode (two kv heads per 4-wave workgroup, pages staged in LDS): workgroup x runs
// the page-range plan's workgroups 2 x and 2 x + 1.
template <class C>
__global__ __launch_bounds__(2 * C::NT) void decode_pair_kernel(BalArgs a) {
    __shared__ PairShared<C> S;
    pair_body<C>(a, S, blockIdx.x);
}

// The reference-shaped uniform split on the balanced body (items of equal key ranges, descriptors
// built in the kernel from the device page table).
template <class C>
__global__ __launch_bounds__(C::NT) void decode_uniform_kernel(UniArgs u) {
    __shared__ BalShared<C, (C::G > 4)> S;   // G = 8: compact, two workgroups per CU (as above)
    balanced_body<C, true, (C::G > 4)>(u.d, S, blockIdx.x, &u);
}

// The drop-in decode_attention over page ranges found on the device (G = 8: the compact layout,
// two workgroups per CU, as for the plan path).
template <class C>
__global__ __launch_bounds__(C::NT) void decode_ranges_kernel(DevArgs d) {
    __shared__ DevShared<C, (C::G > 4)> S;
    dev_body<C, (C::G > 4)>(d, S, blockIdx.x);
}

// The fused cascade step: blocks [0, n_dec) are the suffix decode's workgroups, the rest the
// prefix pass's (item x, kv head) workgroups. Both roles are 4-wave workgroups of about 210
// VGPRs and 69 KB of LDS, so a CU holds one of each: the dispatcher places the first n_dec blocks
// one per CU, and the prefix blocks fill the second slots, so every CU streams suffix pages
// while its matrix core works on the prefix. Partials of both go to the workspace and are merged
// by the next launch.
template <class C, bool RANGES>
__global__ __launch_bounds__(C::NT, 2) void cascade_step_kernel(StepArgs s) {
    static_assert(C::NT == kPrefixThreads, "both roles use the same workgroup shape");
    typedef BalShared<C, (C::G > 4)> Dec;   // G = 8: the compact layout (fits beside a prefix workgroup)
    constexpr size_t SB = sizeof(Dec) > sizeof(PSmem) ? sizeof(Dec) : sizeof(PSmem);
    __shared__ __align__(16) unsigned char raw[SB];
    const int i = blockIdx.x;
    if (i < s.n_dec) {
        balanced_body<C, false, (C::G > 4), RANGES>(s.d, *reinterpret_cast<Dec*>(raw), i);
    } else {
        const int j = i - s.n_dec, n_items = s.p.num_chunks;
        prefix_workgroup(s.p, *reinterpret_cast<PSmem*>(raw), j % n_items, 0, j / n_items);
    }
}

int occupancy_of(const void* fn, int threads) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, 0) != hipSuccess) return 1;
    return n > 0 ? n : 1;
}

// Kernel shapes per group size G.
// One-chunk-per-workgroup kernel (the uniform split's fallback for chunks past the LDS page list):
// 16 lanes per 256-byte row, 4 waves, a two-page ring. Against 8 lanes per row and 8 waves (the
// planner then picks half the chunks, by occupancy), measured cold when it ran every uniform
// split: 64x1K 57.0 vs 64.3 us, 1x32K 39.9 vs 39.8 us, 8x8K 57.2 vs 57.8 us.
template <int G>
using PartialCfg = Cfg<G, 16, 4, 2>;
// Balanced body (plan/run, the uniform split and the cascade's suffix): 4 waves (one per SIMD,
// one workgroup per CU), 16 lanes per row (four row groups per wave, so the end-of-segment merge
// is two permlane steps), a two-page ring: one page in flight while the other is computed. Deeper
// rings measured slower at every shape (4 pages: 30.6 vs 28.5 us back to back at 1x32K, 46.1 vs
// 44.9 us at 64x1K; at G = 8, 3 pages: 29.3 vs 28.6 us and 42.8 vs 41.4 us): more bytes in
// flight only lengthen the memory queues.
template <int G>
using BalCfg = Cfg<G, 16, 4, 2>;
// Paired decode: each kv head's half of the workgroup is two waves (the workgroup is still four
// waves, one per SIMD), a two-page ring per wave in LDS.
template <int G>
using PairCfg = Cfg<G, 16, 2, 2>;

template <class C>
void launch_p(const PartialArgs& a, hipStream_t s) {
    decode_partial_kernel<C><<<dim3(a.num_chunks, a.B * a.Hkv), C::NT, 0, s>>>(a);
}
template <class C>
void launch_b(const BalArgs& a, hipStream_t s) {
    if (a.ngroups > 0) decode_balanced_kernel<C, true><<<a.W, C::NT, 0, s>>>(a);
    else decode_balanced_kernel<C, false><<<a.W, C::NT, 0, s>>>(a);
}
template <class C>
void launch_pair(const BalArgs& a, hipStream_t s) {
    decode_pair_kernel<C><<<a.W / 2, 2 * C::NT, 0, s>>>(a);
}
template <class C>
void launch_u(const UniArgs& a, hipStream_t s) {
    decode_uniform_kernel<C><<<a.d.W, C::NT, 0, s>>>(a);
}
template <class C>
void launch_step(const StepArgs& a, hipStream_t s) {
    if (a.d.ngroups > 0) cascade_step_kernel<C, true><<<a.n_dec + a.n_pre, C::NT, 0, s>>>(a);
    else cascade_step_kernel<C, false><<<a.n_dec + a.n_pre, C::NT, 0, s>>>(a);
}
template <class C>
void launch_r(const DevArgs& a, hipStream_t s) {
    decode_ranges_kernel<C><<<a.d.W, C::NT, 0, s>>>(a);
}
template <class C>
int occ_step() { return occupancy_of(reinterpret_cast<const void*>(&cascade_step_kernel<C, true>), C::NT); }
template <class C>
int occ_p() { return occupancy_of(reinterpret_cast<const void*>(&decode_partial_kernel<C>), C::NT); }
template <class C>
int occ_b() { return occupancy_of(reinterpret_cast<const void*>(&decode_balanced_kernel<C, true>), C::NT); }

#define PD_DISPATCH(CFG, G, FN, ...)                         \
    do {                                                     \
        if ((G) == 1) FN<CFG<1>>(__VA_ARGS__);               \
        else if ((G) == 2) FN<CFG<2>>(__VA_ARGS__);          \
        else if ((G) == 4) FN<CFG<4>>(__VA_ARGS__);          \
        else FN<CFG<8>>(__VA_ARGS__);                        \
    } while (0)

#define PD_DISPATCH_RET(CFG, G, FN)                          \
    do {                                                     \
        if ((G) == 1) return FN<CFG<1>>();                   \
        if ((G) == 2) return FN<CFG<2>>();                   \
        if ((G) == 4) return FN<CFG<4>>();                   \
        return FN<CFG<8>>();                                 \
    } while (0)

}  // namespace

hipError_t launch_decode_partial(const PartialArgs& a, int G, hipStream_t s) {
    if (G != 1 && G != 2 && G != 4 && G != 8) return hipErrorInvalidValue;
    PD_DISPATCH(PartialCfg, G, launch_p, a, s);
    return hipGetLastError();
}

hipError_t launch_merge_states(const float* part_o, const float* part_lse, _Float16* out,
                               float* lse, int rows, int num_chunks, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    merge_states_kernel<<<rows, kMergeThreads, 0, s>>>(part_o, part_lse, out, lse, num_chunks);
    return hipGetLastError();
}

hipError_t launch_decode_balanced(const BalArgs& a, int G, hipStream_t s) {
    if (G != 1 && G != 2 && G != 4 && G != 8) return hipErrorInvalidValue;
    PD_DISPATCH(BalCfg, G, launch_b, a, s);
    return hipGetLastError();
}

hipError_t launch_decode_pair(const BalArgs& a, int G, hipStream_t s) {
    if (G != 1 && G != 2 && G != 4) return hipErrorInvalidValue;
    if (a.ngroups <= 0 || a.Hkv % 2 != 0 || a.W % 2 != 0 || a.W <= 0) return hipErrorInvalidValue;
    if (G == 1) launch_pair<PairCfg<1>>(a, s);
    else if (G == 2) launch_pair<PairCfg<2>>(a, s);
    else launch_pair<PairCfg<4>>(a, s);
    return hipGetLastError();
}

hipError_t launch_decode_uniform(const UniArgs& a, int G, hipStream_t s) {
    if (G != 1 && G != 2 && G != 4 && G != 8) return hipErrorInvalidValue;
    if (a.d.W <= 0) return hipSuccess;
    PD_DISPATCH(BalCfg, G, launch_u, a, s);
    return hipGetLastError();
}

hipError_t launch_cascade_step(const StepArgs& a, int G, hipStream_t s) {
    if (G != 1 && G != 2 && G != 4 && G != 8) return hipErrorInvalidValue;
    if (a.n_dec + a.n_pre <= 0) return hipSuccess;
    PD_DISPATCH(BalCfg, G, launch_step, a, s);
    return hipGetLastError();
}

int occupancy_cascade_step(int G) { PD_DISPATCH_RET(BalCfg, G, occ_step); }

hipError_t launch_merge_split(const MergeArgs& a, int n_entries, hipStream_t s) {
    if (n_entries <= 0) return hipSuccess;
    if (a.cmax > 0) merge_split_kernel<true><<<n_entries * a.G, kMergeThreads, 0, s>>>(a);
    else merge_split_kernel<false><<<n_entries * a.G, kMergeThreads, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_decode_ranges(const DevArgs& a, int G, hipStream_t s) {
    if (G != 1 && G != 2 && G != 4 && G != 8) return hipErrorInvalidValue;
    if (a.d.W <= 0) return hipSuccess;
    PD_DISPATCH(BalCfg, G, launch_r, a, s);
    return hipGetLastError();
}

hipError_t launch_merge_ranges(const DevMergeArgs& a, hipStream_t s) {
    if (a.B <= 0) return hipSuccess;
    merge_ranges_kernel<<<a.B * a.Hq, kMergeThreads, 0, s>>>(a);
    return hipGetLastError();
}

int occupancy_decode_partial(int G) { PD_DISPATCH_RET(PartialCfg, G, occ_p); }
int occupancy_decode_balanced(int G) { PD_DISPATCH_RET(BalCfg, G, occ_b); }

}  // namespace pdattn
