// decode.hip -- paged split-KV GQA decode attention for gfx950 (CDNA4, wave64).
//
// What it computes (qilem/cuda-kernel-lab, 01_decode_attention.cu:76-255): for each sequence b,
// kv head kvh and each of the G query heads h sharing it, over a range of keys,
//   s_j = sm_scale * q_h . k_j,   o = sum_j softmax(s)_j v_j,   lse = ln sum_j exp(s_j)
// as a normalized partial (o, lse), then a log-sum-exp merge of the partials.
//
// How it maps to CDNA4:
//  * A workgroup is 4 waves; all of them work on one (sequence, kv head) token range, each wave
//    on every 4th page of it. K and V rows go straight from HBM into VGPRs with 16-byte loads:
//    a 256-byte row (128 fp16) is read by LPR lanes, so one wave-wide load instruction reads
//    64/LPR rows of one page, each as whole 128-byte lines. No LDS staging is needed because
//    every lane reads only the bytes it computes with.
//  * Scores: each lane takes the fp16 dot product of its slice of q_h and k_j with
//    v_dot2_f32_f16 (fp32 accumulate), then the LPR lanes of a row sum with DPP row ops
//    (quad_perm, row_half_mirror, row_mirror), which leaves the score in every lane of the row.
//  * Every lane therefore owns whole keys: it keeps its own online-softmax state (max, sum,
//    output slice) over the keys it holds, so the PV product needs no cross-lane traffic. The
//    64/LPR independent states of a wave are merged once at the end with shuffles, and the four
//    waves of the workgroup through LDS.
//  * Softmax runs in base 2 on log2(e)-prescaled scores with v_exp_f32 / v_log_f32
//    (exp(x) = 2^(x log2 e)); the running output is rescaled only when some lane's max grows
//    (a wave-uniform branch), which after the first pages is rare.
//  * Prefetch: the loads of the next page are issued before the current page is computed.
//
// Lane geometry, G = query heads per kv head:
//   G <= 4: LPR = 8 lanes per row, 8 rows per load, each lane holds 2 rows x 16 dims of a page;
//   G == 8: LPR = 16, 4 rows per load, each lane holds 4 rows x 8 dims (keeps the fp32 output
//           state at 64 VGPRs).
// Lane (r = lane / LPR, c = lane % LPR) holds rows i*RPI + r of each page and the 16-byte pieces
// kk*LPR + c (dims 8*(kk*LPR + c) .. +7), kk < PPL.
#include <math.h>

#include <algorithm>

#include "pdattn_internal.h"

namespace pdattn {
namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;
constexpr int NW = kDecodeWaves;
constexpr int NT = kDecodeThreads;

template <int G>
struct Geo {
    static constexpr int LPR = (G >= 8) ? 16 : 8;  // lanes per 256-byte K/V row
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

// Reinterprets one 32-bit word as two fp16. The word is taken by value: bit-casting an
// ext-vector element expression in place was observed to read element 0 for every index.
__device__ __forceinline__ f16x2 as_h2(uint32_t w) { return __builtin_bit_cast(f16x2, w); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

template <int G>
struct WaveState {
    float m[G];                   // running max, log2 units
    float l[G];                   // running sum of 2^(x - m)
    float o[G][Geo<G>::DPL];      // running unnormalized output slice
};

template <int G>
struct PageRegs {
    u32x4 k[Geo<G>::RG][Geo<G>::PPL];
    u32x4 v[Geo<G>::RG][Geo<G>::PPL];
};

template <int G>
struct Smem {
    float m[NW][G];
    float l[NW][G];
    float o[NW][G][kHeadDim];
    float fo[G][kHeadDim];    // combined, normalized output of the workgroup
    float flse[G];            // combined lse (natural log)
};

template <int G>
__device__ __forceinline__ void load_page(PageRegs<G>& pr, const uint8_t* kp, const uint8_t* vp,
                                          uint32_t lbase, uint32_t rstride) {
    using g = Geo<G>;
#pragma unroll
    for (int i = 0; i < g::RG; ++i)
#pragma unroll
        for (int kk = 0; kk < g::PPL; ++kk) {
            const uint32_t off = lbase + i * rstride + kk * (g::LPR * 16);
            pr.k[i][kk] = *reinterpret_cast<const u32x4*>(kp + off);
            pr.v[i][kk] = *reinterpret_cast<const u32x4*>(vp + off);
        }
}

// One page: scores, online-softmax update, PV accumulation. tok_r is the token index of this
// lane's row in row group 0; keys outside [tb, te) are masked.
template <int G>
__device__ __forceinline__ void page_step(WaveState<G>& st, const PageRegs<G>& pr,
                                          const f16x2 (&qv)[G][Geo<G>::PPL][4], int tok_r,
                                          int tb, int te, float scale2) {
    using g = Geo<G>;
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

// Attention of the G query heads of (b, kvh) over keys [t0, t1) of one sequence whose page list
// starts at `pages`. Leaves the normalized output in sm.fo and the lse in sm.flse (all threads
// of the workgroup must call it; it ends with a barrier).
template <int G>
__device__ __forceinline__ void process_range(Smem<G>& sm, const _Float16* qrow, const uint8_t* kbase,
                              const uint8_t* vbase, const int32_t* pages, int t0, int t1,
                              int Hkv, int kvh, float scale2) {
    using g = Geo<G>;
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

    WaveState<G> st;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        st.m[h] = -INFINITY;
        st.l[h] = 0.f;
#pragma unroll
        for (int d = 0; d < g::DPL; ++d) st.o[h][d] = 0.f;
    }

    if (t1 > t0) {
        const int pfirst = t0 / kPage, plast = (t1 - 1) / kPage;
        const int npg = plast - pfirst + 1;
        const int nmine = npg > wave ? (npg - wave + NW - 1) / NW : 0;
        const size_t page_bytes = (size_t)kPage * Hkv * 256;
        const uint32_t lbase = (uint32_t)((r * Hkv + kvh) * 256 + c * 16);
        const uint32_t rstride = (uint32_t)(g::RPI * Hkv * 256);
        for (int base = 0; base < nmine; base += 64) {
            const int cnt = min(64, nmine - base);
            // lane j holds the physical page of this wave's (base + j)-th page
            const int pidv = lane < cnt ? pages[pfirst + wave + NW * (base + lane)] : 0;
            PageRegs<G> A, Bf;
            {
                const size_t pid = (uint32_t)__builtin_amdgcn_readlane(pidv, 0);
                load_page<G>(A, kbase + pid * page_bytes, vbase + pid * page_bytes, lbase, rstride);
            }
            for (int it = 0; it < cnt; it += 2) {
                {
                    // prefetch page it+1 (the last page again when there is none: an L2 hit)
                    const int nx = min(it + 1, cnt - 1);
                    const size_t pid = (uint32_t)__builtin_amdgcn_readlane(pidv, nx);
                    load_page<G>(Bf, kbase + pid * page_bytes, vbase + pid * page_bytes, lbase, rstride);
                }
                page_step<G>(st, A, qv, (pfirst + wave + NW * (base + it)) * kPage + r, t0, t1, scale2);
                if (it + 1 >= cnt) break;
                {
                    const int nx = min(it + 2, cnt - 1);
                    const size_t pid = (uint32_t)__builtin_amdgcn_readlane(pidv, nx);
                    load_page<G>(A, kbase + pid * page_bytes, vbase + pid * page_bytes, lbase, rstride);
                }
                page_step<G>(st, Bf, qv, (pfirst + wave + NW * (base + it + 1)) * kPage + r, t0, t1, scale2);
            }
        }
    }

    // merge the 64/LPR row-group states of this wave (lanes LPR apart hold the same dims)
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float M = st.m[h];
#pragma unroll
        for (int off = g::LPR; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float a = (st.m[h] == -INFINITY) ? 0.f : fast_exp2(st.m[h] - M);
        float l = st.l[h] * a;
#pragma unroll
        for (int off = g::LPR; off < 64; off <<= 1) l += __shfl_xor(l, off);
#pragma unroll
        for (int d = 0; d < g::DPL; ++d) {
            float v = st.o[h][d] * a;
#pragma unroll
            for (int off = g::LPR; off < 64; off <<= 1) v += __shfl_xor(v, off);
            st.o[h][d] = v;
        }
        st.m[h] = M;
        st.l[h] = l;
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
    for (int idx = tid; idx < G * kHeadDim; idx += NT) {
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

// ---- uniform chunks: the reference's decode_partial launch shape -------------------------
template <int G>
__global__ __launch_bounds__(NT) void decode_partial_kernel(PartialArgs a) {
    __shared__ Smem<G> sm;
    const int chunk = blockIdx.x;
    const int b = blockIdx.y / a.Hkv, kvh = blockIdx.y % a.Hkv;
    const int pb = a.kv_indptr[b];
    const int np = a.kv_indptr[b + 1] - pb;
    const int len = np > 0 ? (np - 1) * kPage + a.kv_last[b] : 0;
    const int kbeg = a.kv_start + chunk * a.chunk_tokens;
    const int kend = min(len, kbeg + a.chunk_tokens);
    process_range<G>(sm, a.q + ((size_t)b * a.Hq + kvh * G) * kHeadDim, a.k, a.v,
                     a.kv_indices + pb, kbeg, kend, a.Hkv, kvh, a.scale_log2);
    for (int idx = threadIdx.x; idx < G * kHeadDim; idx += NT) {
        const int h = idx / kHeadDim, d = idx % kHeadDim;
        const size_t slot = ((size_t)b * a.Hq + kvh * G + h) * a.part_stride + a.chunk_base + chunk;
        a.part_o[slot * kHeadDim + d] = sm.fo[h][d];
        if (d == 0) a.part_lse[slot] = sm.flse[h];
    }
}

// ---- log-sum-exp merge: the reference's merge_states launch shape -------------------------
__global__ __launch_bounds__(kHeadDim) void merge_states_kernel(const float* __restrict__ part_o,
                                                                 const float* __restrict__ part_lse,
                                                                 _Float16* __restrict__ out,
                                                                 float* __restrict__ lse_out,
                                                                 int num_chunks) {
    const int row = blockIdx.x, t = threadIdx.x;
    const float* pl = part_lse + (size_t)row * num_chunks;
    float m = -INFINITY;
    for (int c = 0; c < num_chunks; ++c) m = fmaxf(m, pl[c]);
    float ws = 0.f, acc = 0.f;
    if (m != -INFINITY) {
        const float* po = part_o + (size_t)row * num_chunks * kHeadDim + t;
        for (int c = 0; c < num_chunks; ++c) {
            const float w = fast_exp2((pl[c] - m) * kLog2e);
            ws += w;
            acc = fmaf(w, po[(size_t)c * kHeadDim], acc);
        }
    }
    out[(size_t)row * kHeadDim + t] = (_Float16)(ws > 0.f ? acc / ws : 0.f);
    if (t == 0) lse_out[row] = ws > 0.f ? m + fast_log2(ws) * kLn2 : -INFINITY;
}

// ---- balanced single launch ------------------------------------------------------------------
// Combines `n` stored partial states (natural-log lse) of one row plus the row's extra partials,
// in fixed order, and writes fp16 out / fp32 lse. `own_o/own_lse` (if own_valid) is one more
// state taken from LDS, placed first.
template <int G>
__device__ __forceinline__ void combine_row(const StreamKArgs& a, size_t row, int h, int d,
                                            bool own_valid, float own_o, float own_lse,
                                            const float* slot_o, const float* slot_lse,
                                            int nslots) {
    float m = own_valid ? own_lse : -INFINITY;
    for (int k = 0; k < nslots; ++k) m = fmaxf(m, slot_lse[(size_t)k * G]);
    const float* eo = a.extra_o + row * (size_t)a.extra_stride * kHeadDim;
    const float* el = a.extra_lse + row * (size_t)a.extra_stride;
    for (int e = 0; e < a.n_extra; ++e) m = fmaxf(m, el[e]);
    float ws = 0.f, acc = 0.f;
    if (m != -INFINITY) {
        if (own_valid && own_lse != -INFINITY) {
            const float w = fast_exp2((own_lse - m) * kLog2e);
            ws += w;
            acc = fmaf(w, own_o, acc);
        }
        for (int k = 0; k < nslots; ++k) {
            const float lk = slot_lse[(size_t)k * G];
            if (lk == -INFINITY) continue;
            const float w = fast_exp2((lk - m) * kLog2e);
            ws += w;
            acc = fmaf(w, slot_o[(size_t)k * G * kHeadDim], acc);
        }
        for (int e = 0; e < a.n_extra; ++e) {
            if (el[e] == -INFINITY) continue;
            const float w = fast_exp2((el[e] - m) * kLog2e);
            ws += w;
            acc = fmaf(w, eo[(size_t)e * kHeadDim + d], acc);
        }
    }
    a.out[row * kHeadDim + d] = (_Float16)(ws > 0.f ? acc / ws : 0.f);
    if (d == 0) a.lse[row] = ws > 0.f ? m + fast_log2(ws) * kLn2 : -INFINITY;
    (void)h;
}

template <int G>
__global__ __launch_bounds__(NT) void decode_streamk_kernel(StreamKArgs a) {
    __shared__ Smem<G> sm;
    __shared__ int s_last;
    const int w = blockIdx.x, tid = threadIdx.x;

    // Sequences without pages: the result is the merge of the extra partials alone (0 / -inf
    // when there are none).
    for (int rr = w; rr < a.n_empty * a.Hq; rr += a.W) {
        const size_t row = (size_t)a.empty_seq[rr / a.Hq] * a.Hq + rr % a.Hq;
        for (int d = tid; d < kHeadDim; d += NT)
            combine_row<G>(a, row, 0, d, false, 0.f, -INFINITY, nullptr, nullptr, 0);
    }

    const int64_t u1 = a.U * (w + 1) / a.W;
    int64_t u = a.U * w / a.W;
    if (u >= u1) return;
    int kvh = (int)(u / a.nnz);
    int j = (int)(u - (int64_t)kvh * a.nnz);
    int b = a.desc_b0[w];
    while (true) {
        const int pb = a.kv_indptr[b] - a.jbase, pe = a.kv_indptr[b + 1] - a.jbase;
        const int len = (pe - pb - 1) * kPage + a.kv_last[b];
        const int je = (int)min((int64_t)pe, (int64_t)j + (u1 - u));
        const int t0 = (j - pb) * kPage;
        const int t1 = min(len, (je - pb) * kPage);
        process_range<G>(sm, a.q + ((size_t)b * a.Hq + kvh * G) * kHeadDim, a.k, a.v,
                         a.kv_indices + a.jbase + pb, t0, t1, a.Hkv, kvh, a.scale_log2);
        if (j == pb && je == pe) {
            // the whole (sequence, kv head) pair was ours: final result
            for (int idx = tid; idx < G * kHeadDim; idx += NT) {
                const int h = idx / kHeadDim, d = idx % kHeadDim;
                const size_t row = (size_t)b * a.Hq + kvh * G + h;
                if (a.n_extra == 0) {
                    a.out[row * kHeadDim + d] = (_Float16)sm.fo[h][d];
                    if (d == 0) a.lse[row] = sm.flse[h];
                } else {
                    combine_row<G>(a, row, h, d, true, sm.fo[h][d], sm.flse[h], nullptr, nullptr, 0);
                }
            }
        } else {
            // one of several contributors: store the partial, count arrivals; the last merges
            const int p = kvh * a.B + b;
            const int64_t ufirst = (int64_t)kvh * a.nnz + pb, ulast = ufirst + (pe - pb) - 1;
            const int w1 = (int)(((ufirst + 1) * a.W - 1) / a.U);
            const int w2 = (int)(((ulast + 1) * a.W - 1) / a.U);
            const size_t slot = (size_t)p + w;
            for (int idx = tid; idx < G * kHeadDim; idx += NT) {
                const int h = idx / kHeadDim, d = idx % kHeadDim;
                a.part_o[(slot * G + h) * kHeadDim + d] = sm.fo[h][d];
                if (d == 0) a.part_lse[slot * G + h] = sm.flse[h];
            }
            __threadfence();
            __syncthreads();
            if (tid == 0) {
                const int old = atomicAdd(&a.counters[p], 1);
                s_last = (old == w2 - w1) ? 1 : 0;
            }
            __syncthreads();
            if (s_last) {
                __threadfence();
                const size_t s0 = (size_t)p + w1;
                for (int idx = tid; idx < G * kHeadDim; idx += NT) {
                    const int h = idx / kHeadDim, d = idx % kHeadDim;
                    const size_t row = (size_t)b * a.Hq + kvh * G + h;
                    combine_row<G>(a, row, h, d, false, 0.f, -INFINITY,
                                   a.part_o + (s0 * G + h) * kHeadDim + d, a.part_lse + s0 * G + h,
                                   w2 - w1 + 1);
                }
                if (tid == 0) atomicExch(&a.counters[p], 0);
            }
        }
        u += je - j;
        j = je;
        if (u >= u1) break;
        if (j == a.nnz) {
            ++kvh;
            j = 0;
            b = a.b_first;
        } else {
            ++b;
            while (a.kv_indptr[b + 1] == a.kv_indptr[b]) ++b;
        }
        __syncthreads();  // sm is reused by the next segment
    }
}

__global__ void fill_i32_kernel(int32_t* p, int32_t value, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = value;
}

template <int G>
const void* partial_kernel_ptr() { return reinterpret_cast<const void*>(&decode_partial_kernel<G>); }
template <int G>
const void* streamk_kernel_ptr() { return reinterpret_cast<const void*>(&decode_streamk_kernel<G>); }

int occupancy_of(const void* fn, int threads) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, 0) != hipSuccess) return 1;
    return n > 0 ? n : 1;
}

}  // namespace

hipError_t launch_decode_partial(const PartialArgs& a, int G, hipStream_t s) {
    dim3 grid(a.num_chunks, a.B * a.Hkv);
    switch (G) {
        case 1: decode_partial_kernel<1><<<grid, NT, 0, s>>>(a); break;
        case 2: decode_partial_kernel<2><<<grid, NT, 0, s>>>(a); break;
        case 4: decode_partial_kernel<4><<<grid, NT, 0, s>>>(a); break;
        case 8: decode_partial_kernel<8><<<grid, NT, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_merge_states(const float* part_o, const float* part_lse, _Float16* out,
                               float* lse, int rows, int num_chunks, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    merge_states_kernel<<<rows, kHeadDim, 0, s>>>(part_o, part_lse, out, lse, num_chunks);
    return hipGetLastError();
}

hipError_t launch_decode_streamk(const StreamKArgs& a, int G, hipStream_t s) {
    switch (G) {
        case 1: decode_streamk_kernel<1><<<a.W, NT, 0, s>>>(a); break;
        case 2: decode_streamk_kernel<2><<<a.W, NT, 0, s>>>(a); break;
        case 4: decode_streamk_kernel<4><<<a.W, NT, 0, s>>>(a); break;
        case 8: decode_streamk_kernel<8><<<a.W, NT, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_fill_i32(int32_t* p, int32_t value, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const int grid = (int)std::min<size_t>((n + 255) / 256, 1024);
    fill_i32_kernel<<<grid, 256, 0, s>>>(p, value, n);
    return hipGetLastError();
}

int occupancy_decode_partial(int G) {
    switch (G) {
        case 1: return occupancy_of(partial_kernel_ptr<1>(), NT);
        case 2: return occupancy_of(partial_kernel_ptr<2>(), NT);
        case 4: return occupancy_of(partial_kernel_ptr<4>(), NT);
        default: return occupancy_of(partial_kernel_ptr<8>(), NT);
    }
}

int occupancy_decode_streamk(int G) {
    switch (G) {
        case 1: return occupancy_of(streamk_kernel_ptr<1>(), NT);
        case 2: return occupancy_of(streamk_kernel_ptr<2>(), NT);
        case 4: return occupancy_of(streamk_kernel_ptr<4>(), NT);
        default: return occupancy_of(streamk_kernel_ptr<8>(), NT);
    }
}

}  // namespace pdattn
