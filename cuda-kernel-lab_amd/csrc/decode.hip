// decode.hip -- paged split-KV GQA decode attention for gfx950 (CDNA4, wave64).
//
// What it computes (qilem/cuda-kernel-lab, 01_decode_attention.cu:76-255): for each sequence b,
// kv head kvh and each of the G query heads h sharing it, over a range of keys,
//   s_j = sm_scale * q_h . k_j,   o = sum_j softmax(s)_j v_j,   lse = ln sum_j exp(s_j)
// as a normalized partial (o, lse), then a log-sum-exp merge of the partials.
//
// How it maps to CDNA4:
//  * A workgroup is 8 waves; all of them work on one (sequence, kv head) token range, each wave
//    on every 8th page of it. K and V rows go straight from HBM into VGPRs with 16-byte
//    non-temporal loads: a 256-byte row (128 fp16) is read by LPR lanes, so one wave-wide load
//    instruction reads 64/LPR rows of one page, each as whole 128-byte lines. No LDS staging is
//    needed because every lane reads only the bytes it computes with.
//  * Scores: each lane takes the fp16 dot product of its slice of q_h and k_j with
//    v_dot2_f32_f16 (fp32 accumulate), then the LPR lanes of a row sum with DPP row ops
//    (quad_perm, row_half_mirror, row_mirror), which leaves the score in every lane of the row.
//  * Every lane therefore owns whole keys: it keeps its own online-softmax state (max, sum,
//    output slice) over the keys it holds, so the PV product needs no cross-lane traffic. The
//    64/LPR independent states of a wave are merged once at the end in the VALU (DPP row_ror and
//    v_permlane16/32_swap), and the eight waves of the workgroup through LDS.
//  * Softmax runs in base 2 on log2(e)-prescaled scores with v_exp_f32 / v_log_f32
//    (exp(x) = 2^(x log2 e)); the running output is rescaled only when some lane's max grows
//    (a wave-uniform branch), which after the first pages is rare.
//  * Prefetch: a two-page ring in VGPRs; the loads of the next page are issued before the
//    current page is computed.
//
// Lane geometry, G = query heads per kv head:
//   G <= 4: LPR = 8 lanes per row, 8 rows per load, each lane holds 2 rows x 16 dims of a page;
//   G == 8: LPR = 16, 4 rows per load, each lane holds 4 rows x 8 dims (keeps the fp32 output
//           state at 64 VGPRs).
// Lane (r = lane / LPR, c = lane % LPR) holds rows i*RPI + r of each page and the 16-byte pieces
// kk*LPR + c (dims 8*(kk*LPR + c) .. +7), kk < PPL.
#include <math.h>

#include <algorithm>
#include <cstdlib>

#include "pdattn_internal.h"

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

// Combine of the 64/LPR row groups of a wave (lanes LPR apart hold the same head dims), leaving
// the result in every lane: row_ror:8 pairs the two groups of a 16-lane row (LPR = 8), then
// v_permlane16_swap / v_permlane32_swap pair whole 16-lane rows, all in the VALU. After
// swap(a, b) the two results hold, in every lane, the values of both rows of its pair (rows
// r and r^1 for the 16-lane swap, r and r^2 for the 32-lane swap), always in the same order, so
// r0 + r1 is bitwise the same in all lanes. The second operand is passed through an empty asm
// statement: given the same SSA value twice, the compiler treats the two results as equal and
// drops the second one.
__device__ __forceinline__ unsigned opaque_copy(unsigned v) {
    asm volatile("" : "+v"(v));
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
    float wmax[NW][G];        // merge scratch: per-wave maxima,
    float gmax[G];            //   per-row maximum,
    float red[NW * 64 * 6];   //   per-thread partial states
};

template <class C>
__device__ __forceinline__ void load_page(PageRegs<C>& pr, const uint8_t* kp, const uint8_t* vp,
                                          uint32_t lbase, uint32_t rstride) {
    using g = C;
#pragma unroll
    for (int i = 0; i < g::RG; ++i)
#pragma unroll
        for (int kk = 0; kk < g::PPL; ++kk) {
            const uint32_t off = lbase + i * rstride + kk * (g::LPR * 16);
            // K/V bytes are read exactly once: non-temporal loads keep them from displacing
            // reusable lines in L2 and the Infinity Cache
            pr.k[i][kk] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + off));
            pr.v[i][kk] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vp + off));
        }
}

// One page: scores, online-softmax update, PV accumulation. tok_r is the token index of this
// lane's row in row group 0; keys outside [tb, te) are masked.
template <class C>
__device__ __forceinline__ void page_step(WaveState<C>& st, const PageRegs<C>& pr,
                                          const f16x2 (&qv)[C::G][C::PPL][4], int tok_r,
                                          int tb, int te, float scale2) {
    using g = C;
    constexpr int G = C::G;
    float x[g::RG][G];
#pragma unroll
    for (int i = 0; i < g::RG; ++i) {
        const int tok = tok_r + i * g::RPI;
        const bool ok = tok >= tb && tok < te;
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
            acc = row_sum<g::LPR>(acc);
            x[i][h] = ok ? acc * scale2 : -INFINITY;
        }
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
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
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
        const size_t page_bytes = (size_t)kPage * Hkv * 256;
        const uint32_t lbase = (uint32_t)((r * Hkv + kvh) * 256 + c * 16);
        const uint32_t rstride = (uint32_t)(g::RPI * Hkv * 256);
        for (int base = 0; base < nmine; base += 64) {
            const int cnt = min(64, nmine - base);
            // lane j holds the physical page of this wave's (base + j)-th page
            const int pidv = lane < cnt ? pages[pfirst + wave + NW * (base + lane)] : 0;
            // ring of NBUF pages in VGPRs: page i lives in buf[i % NBUF]; NBUF-1 are in flight
            // while one is computed. Past the end the last page is loaded again (an L2 hit), so
            // every iteration issues the same loads and the wait counts stay exact.
            PageRegs<C> buf[NBUF];
#pragma unroll
            for (int u = 0; u < NBUF - 1; ++u) {
                const size_t pid = (uint32_t)__builtin_amdgcn_readlane(pidv, min(u, cnt - 1));
                load_page<C>(buf[u], kbase + pid * page_bytes, vbase + pid * page_bytes, lbase, rstride);
            }
            for (int it = 0; it < cnt; it += NBUF) {
#pragma unroll
                for (int u = 0; u < NBUF; ++u) {
                    if (it + u >= cnt) break;
                    {
                        const int nx = min(it + u + NBUF - 1, cnt - 1);
                        const size_t pid = (uint32_t)__builtin_amdgcn_readlane(pidv, nx);
                        load_page<C>(buf[(u + NBUF - 1) % NBUF], kbase + pid * page_bytes,
                                     vbase + pid * page_bytes, lbase, rstride);
                    }
                    page_step<C>(st, buf[u], qv, tok_base + (pfirst + wave + NW * (base + it + u)) * kPage + r,
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
typedef const __attribute__((address_space(4))) StreamKArgs* KArgPtr;
__device__ __forceinline__ KArgPtr kargs() {
    KArgPtr p = (KArgPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return p;
}

// ---- merging partial states ----------------------------------------------------------------
// Online log-sum-exp accumulation of one partial state (lse l, normalized output o) into
// (m, ws, acc): acc / ws is the merged output, m + ln ws the merged lse. Empty states
// (l = -inf) are identities.
__device__ __forceinline__ void lse_accumulate(float& m, float& ws, float4& acc, float l, float4 o) {
    if (l == -INFINITY) return;
    if (l > m) {
        const float sc = fast_exp2((m - l) * kLog2e);   // m = -inf gives 0
        ws *= sc;
        acc.x *= sc;
        acc.y *= sc;
        acc.z *= sc;
        acc.w *= sc;
        m = l;
    }
    const float w = fast_exp2((l - m) * kLog2e);
    ws += w;
    acc.x = fmaf(w, o.x, acc.x);
    acc.y = fmaf(w, o.y, acc.y);
    acc.z = fmaf(w, o.z, acc.z);
    acc.w = fmaf(w, o.w, acc.w);
}

// Log-sum-exp merge of the G rows of one (sequence, kv head) pair from a list of sources, in a
// fixed source order (deterministic whatever order the sources were produced in):
//   source 0 (if `own`): the workgroup's own result in LDS (sm.fo / sm.flse);
//   then `nslots` stored partials: o at part_o[((s0 + k) * G + h) * 128], lse at part_lse[(s0 + k) * G + h];
//   then the `n_extra` extra partials of each row: o at extra_o[(row * n_extra + e) * 128], lse at
//   extra_lse[row * n_extra + e].
// One pass: each thread owns one 4-dim quad of one row and every TPQ-th source, issues all its
// loads, accumulates them online, and the TPQ partial states of a quad are combined in order
// through LDS. Writes fp16 out and fp32 lse; a row whose every source is empty gets 0 / -inf.
template <int G, int NW, bool ACQUIRE>
__device__ __forceinline__ void merge_sources(Smem<G, NW>& sm, KArgPtr a, int b, int kvh, bool own,
                                              int64_t s0, int nslots) {
    // partials written by other workgroups (write-through atomic stores, completed before their
    // arrival was counted): drop any stale copies this XCD's caches hold, then plain loads
    if constexpr (ACQUIRE) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    constexpr int NT = NW * 64;
    constexpr int Q = G * 32;          // 4-dim quads of the G rows
    constexpr int TPQ = NT / Q;        // threads per quad
    static_assert(NT % Q == 0, "thread count must cover the quads");
    const int tid = threadIdx.x;
    const int n_extra = a->n_extra;
    const int nsrc = (own ? 1 : 0) + nslots + n_extra;
    const size_t row0 = (size_t)b * a->Hq + (size_t)kvh * G;
    const int quad = tid % Q, r = tid / Q;
    const int h = quad / 32, d0 = 4 * (quad % 32);

    auto load_src = [&](int k, float& l, float4& o) {
        if (own) {
            if (k == 0) {
                l = sm.flse[h];
                o = make_float4(sm.fo[h][d0], sm.fo[h][d0 + 1], sm.fo[h][d0 + 2], sm.fo[h][d0 + 3]);
                return;
            }
            --k;
        }
        if (k < nslots) {
            const float* pl = a->part_lse + (s0 + k) * G + h;
            const float* po = a->part_o + ((s0 + k) * G + h) * kHeadDim + d0;
            l = *pl;
            o = *reinterpret_cast<const float4*>(po);
            return;
        }
        const size_t e = (row0 + h) * n_extra + (k - nslots);
        l = a->extra_lse[e];
        o = *reinterpret_cast<const float4*>(a->extra_o + e * kHeadDim + d0);
    };

    float m = -INFINITY, ws = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = r; k < nsrc; k += 4 * TPQ) {
        float l[4];
        float4 o[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) load_src(min(k + u * TPQ, nsrc - 1), l[u], o[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (k + u * TPQ < nsrc) lse_accumulate(m, ws, acc, l[u], o[u]);
    }
    float* red = sm.red + (size_t)tid * 6;
    red[0] = m;
    red[1] = ws;
    red[2] = acc.x;
    red[3] = acc.y;
    red[4] = acc.z;
    red[5] = acc.w;
    __syncthreads();
    if (r == 0) {
        for (int rr = 1; rr < TPQ; ++rr) {
            const float* o = sm.red + (size_t)(rr * Q + quad) * 6;
            if (o[1] > 0.f) {
                // fold in a partial state (o[0] + ln o[1], o[2..5] / o[1])
                const float mm = fmaxf(m, o[0]);
                const float sa = fast_exp2((m - mm) * kLog2e), sb = fast_exp2((o[0] - mm) * kLog2e);
                ws = ws * sa + o[1] * sb;
                acc.x = acc.x * sa + o[2] * sb;
                acc.y = acc.y * sa + o[3] * sb;
                acc.z = acc.z * sa + o[4] * sb;
                acc.w = acc.w * sa + o[5] * sb;
                m = mm;
            }
        }
        const float inv = ws > 0.f ? 1.f / ws : 0.f;
        _Float16* out = a->out + (row0 + h) * kHeadDim + d0;
        out[0] = (_Float16)(acc.x * inv);
        out[1] = (_Float16)(acc.y * inv);
        out[2] = (_Float16)(acc.z * inv);
        out[3] = (_Float16)(acc.w * inv);
        if (d0 == 0) a->lse[row0 + h] = ws > 0.f ? m + fast_log2(ws) * kLn2 : -INFINITY;
    }
    __syncthreads();
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
    const int len = np > 0 ? (np - 1) * kPage + a.kv_last[b] : 0;
    const int kbeg = a.kv_start + chunk * a.chunk_tokens;
    const int kend = min(len, kbeg + a.chunk_tokens);
    process_range<C>(sm, a.q + ((size_t)b * a.Hq + kvh * G) * kHeadDim, a.k, a.v,
                     a.kv_indices + pb, 0, kbeg, kend, a.Hkv, kvh, a.scale_log2);
    for (int idx = threadIdx.x; idx < G * kHeadDim; idx += C::NT) {
        const int h = idx / kHeadDim, d = idx % kHeadDim;
        const size_t slot = ((size_t)b * a.Hq + kvh * G + h) * a.part_stride + a.chunk_base + chunk;
        a.part_o[slot * kHeadDim + d] = sm.fo[h][d];
        if (d == 0) a.part_lse[slot] = sm.flse[h];
    }
}

// ---- log-sum-exp merge: the reference's merge_states launch shape -------------------------
// One workgroup per row: each of 8 threads per 4-dim quad takes every 8th chunk (independent
// 16-byte loads, accumulated online), and the 8 states are combined in order through LDS.
constexpr int kMergeThreads = 256;
__global__ __launch_bounds__(kMergeThreads) void merge_states_kernel(const float* __restrict__ part_o,
                                                                      const float* __restrict__ part_lse,
                                                                      _Float16* __restrict__ out,
                                                                      float* __restrict__ lse_out,
                                                                      int num_chunks) {
    constexpr int Q = kHeadDim / 4, TPQ = kMergeThreads / Q;
    __shared__ float red[kMergeThreads * 6];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* pl = part_lse + (size_t)row * num_chunks;
    const float* po = part_o + (size_t)row * num_chunks * kHeadDim;
    const int quad = tid % Q, r = tid / Q, d0 = 4 * quad;
    float m = -INFINITY, ws = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c = r; c < num_chunks; c += 4 * TPQ) {
        float l[4];
        float4 o[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int cc = min(c + u * TPQ, num_chunks - 1);
            l[u] = pl[cc];
            o[u] = *reinterpret_cast<const float4*>(po + (size_t)cc * kHeadDim + d0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (c + u * TPQ < num_chunks) lse_accumulate(m, ws, acc, l[u], o[u]);
    }
    float* rd = red + tid * 6;
    rd[0] = m;
    rd[1] = ws;
    rd[2] = acc.x;
    rd[3] = acc.y;
    rd[4] = acc.z;
    rd[5] = acc.w;
    __syncthreads();
    if (r == 0) {
        for (int rr = 1; rr < TPQ; ++rr) {
            const float* o = red + (rr * Q + quad) * 6;
            if (o[1] > 0.f) {
                const float mm = fmaxf(m, o[0]);
                const float sa = fast_exp2((m - mm) * kLog2e), sb = fast_exp2((o[0] - mm) * kLog2e);
                ws = ws * sa + o[1] * sb;
                acc.x = acc.x * sa + o[2] * sb;
                acc.y = acc.y * sa + o[3] * sb;
                acc.z = acc.z * sa + o[4] * sb;
                acc.w = acc.w * sa + o[5] * sb;
                m = mm;
            }
        }
        const float inv = ws > 0.f ? 1.f / ws : 0.f;
        _Float16* op = out + (size_t)row * kHeadDim + d0;
        op[0] = (_Float16)(acc.x * inv);
        op[1] = (_Float16)(acc.y * inv);
        op[2] = (_Float16)(acc.z * inv);
        op[3] = (_Float16)(acc.w * inv);
        if (quad == 0) lse_out[row] = ws > 0.f ? m + fast_log2(ws) * kLn2 : -INFINITY;
    }
}

// ---- balanced single launch ------------------------------------------------------------------
// Hand-off of a split pair's partials between workgroups, possibly on different XCDs (whose L2
// caches are not coherent with each other): contributors write their partial with agent-scope
// atomic stores (write-through to the coherent level), wait until those stores have completed
// (s_waitcnt), then count themselves in with an agent-scope atomic add; the last contributor
// invalidates its own caches once (agent-scope acquire) and reads the partials with plain
// vector loads. No L2 write-back (which __threadfence() would issue in every contributing
// workgroup, flushing and invalidating that XCD's whole L2) is needed.
template <class C>
__global__ __launch_bounds__(C::NT) void decode_streamk_kernel(StreamKArgs a) {
    constexpr int G = C::G, NW = C::NW, NT = C::NT;
    __shared__ Smem<G, NW> sm;
    __shared__ int pg[kRangeMax];
    __shared__ int s_last;
    const int w = blockIdx.x, tid = threadIdx.x;

    // Sequences without pages: the result is the merge of the extra partials alone (0 / -inf
    // when there are none).
    for (int e = w; e < kargs()->n_empty * a.Hkv; e += a.W)
        merge_sources<G, NW, false>(sm, kargs(), kargs()->empty_seq[e / a.Hkv], e % a.Hkv, false, 0, 0);

    const int64_t u0 = a.U * w / a.W, u1 = a.U * (w + 1) / a.W;
    const int R = (int)(u1 - u0);
    if (R <= 0) return;
    // page ids of this workgroup's range: units u0 .. u1-1 of the kv-head-major order are the
    // consecutive page-table positions (u mod nnz), so they load before any descriptor arrives
    for (int qq = tid; qq < R; qq += NT)
        pg[qq] = a.kv_indices[a.jbase + (int)((u0 + qq) % a.nnz)];
    const int nseg = kargs()->desc[(size_t)w * kDescInts];
    __syncthreads();

    for (int si = 0; si < nseg; ++si) {
        const int32_t* sg = kargs()->desc + (size_t)w * kDescInts + 8 + kSegInts * si;
        const int b = sg[0], kvh = sg[1], qa = sg[2], t0 = sg[4], t1 = sg[5];
        process_range<C>(sm, a.q + ((size_t)b * a.Hq + kvh * G) * kHeadDim, a.k, a.v, pg + qa, t0,
                         t0, t1, a.Hkv, kvh, a.scale_log2);
        const int32_t* sg2 = kargs()->desc + (size_t)w * kDescInts + 8 + kSegInts * si;
        const int w1 = sg2[6], nc = sg2[7];
        if (nc == 1) {
            // the whole (sequence, kv head) pair was ours: final result
            if (kargs()->n_extra == 0) {
                for (int idx = tid; idx < G * kHeadDim; idx += NT) {
                    const int h = idx / kHeadDim, d = idx % kHeadDim;
                    const size_t row = (size_t)b * a.Hq + kvh * G + h;
                    kargs()->out[row * kHeadDim + d] = (_Float16)sm.fo[h][d];
                    if (d == 0) kargs()->lse[row] = sm.flse[h];
                }
            } else {
                merge_sources<G, NW, false>(sm, kargs(), b, kvh, true, 0, 0);
            }
        } else {
            // one of nc contributors: store the partial with agent-scope atomic stores, count
            // arrivals; the last one merges all nc partials in workgroup order
            const int p = kvh * a.B + b;
            const size_t slot = (size_t)p + w;
            for (int idx = tid; idx < G * kHeadDim; idx += NT) {
                const int h = idx / kHeadDim, d = idx % kHeadDim;
                __hip_atomic_store(kargs()->part_o + (slot * G + h) * kHeadDim + d, sm.fo[h][d],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (d == 0)
                    __hip_atomic_store(kargs()->part_lse + slot * G + h, sm.flse[h], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
            __builtin_amdgcn_s_waitcnt(0);   // this thread's partial stores have completed
            __syncthreads();
            if (tid == 0) {
                const int old = __hip_atomic_fetch_add(&kargs()->counters[p], 1, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
                s_last = (old == nc - 1) ? 1 : 0;
            }
            __syncthreads();
            if (s_last) {
                merge_sources<G, NW, true>(sm, kargs(), b, kvh, false, (int64_t)p + w1, nc);
                if (tid == 0)
                    __hip_atomic_store(&kargs()->counters[p], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();  // sm is reused by the next segment
    }
}

__global__ void fill_i32_kernel(int32_t* p, int32_t value, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = value;
}

int occupancy_of(const void* fn, int threads) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, 0) != hipSuccess) return 1;
    return n > 0 ? n : 1;
}

// Kernel shape per group size G: 8 lanes per 256-byte row (16 for G = 8, which needs the
// registers), 8 waves, and a two-page ring. Deeper rings (3, 4, 6 pages), 16 lanes per row for
// G = 4 and 4-wave workgroups measured within a few percent of this shape on MI355X.
template <int G>
using DefaultCfg = Cfg<G, (G >= 8 ? 16 : 8), 8, 2>;

template <class C>
void launch_p(const PartialArgs& a, hipStream_t s) {
    decode_partial_kernel<C><<<dim3(a.num_chunks, a.B * a.Hkv), C::NT, 0, s>>>(a);
}
template <class C>
void launch_s(const StreamKArgs& a, hipStream_t s) {
    decode_streamk_kernel<C><<<a.W, C::NT, 0, s>>>(a);
}
template <class C>
int occ_p() { return occupancy_of(reinterpret_cast<const void*>(&decode_partial_kernel<C>), C::NT); }
template <class C>
int occ_s() { return occupancy_of(reinterpret_cast<const void*>(&decode_streamk_kernel<C>), C::NT); }

#define PD_DISPATCH(G, FN, ...)                              \
    do {                                                     \
        if ((G) == 1) FN<DefaultCfg<1>>(__VA_ARGS__);        \
        else if ((G) == 2) FN<DefaultCfg<2>>(__VA_ARGS__);   \
        else if ((G) == 4) FN<DefaultCfg<4>>(__VA_ARGS__);   \
        else FN<DefaultCfg<8>>(__VA_ARGS__);                 \
    } while (0)

#define PD_DISPATCH_RET(G, FN)                               \
    do {                                                     \
        if ((G) == 1) return FN<DefaultCfg<1>>();            \
        if ((G) == 2) return FN<DefaultCfg<2>>();            \
        if ((G) == 4) return FN<DefaultCfg<4>>();            \
        return FN<DefaultCfg<8>>();                          \
    } while (0)

}  // namespace

hipError_t launch_decode_partial(const PartialArgs& a, int G, hipStream_t s) {
    if (G != 1 && G != 2 && G != 4 && G != 8) return hipErrorInvalidValue;
    PD_DISPATCH(G, launch_p, a, s);
    return hipGetLastError();
}

hipError_t launch_merge_states(const float* part_o, const float* part_lse, _Float16* out,
                               float* lse, int rows, int num_chunks, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    merge_states_kernel<<<rows, kMergeThreads, 0, s>>>(part_o, part_lse, out, lse, num_chunks);
    return hipGetLastError();
}

hipError_t launch_decode_streamk(const StreamKArgs& a, int G, hipStream_t s) {
    if (G != 1 && G != 2 && G != 4 && G != 8) return hipErrorInvalidValue;
    PD_DISPATCH(G, launch_s, a, s);
    return hipGetLastError();
}

hipError_t launch_fill_i32(int32_t* p, int32_t value, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const int grid = (int)std::min<size_t>((n + 255) / 256, 1024);
    fill_i32_kernel<<<grid, 256, 0, s>>>(p, value, n);
    return hipGetLastError();
}

int occupancy_decode_partial(int G) { PD_DISPATCH_RET(G, occ_p); }
int occupancy_decode_streamk(int G) { PD_DISPATCH_RET(G, occ_s); }

}  // namespace pdattn
