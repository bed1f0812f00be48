// prefix_body.h -- shared-prefix ("cascade") attention on CDNA4 fp16 MFMA: the workgroup body,
// shared by the prefix kernel (cascade.hip) and the fused cascade step (decode.hip).
//
// With prefix caching, all B sequences of a batch start with the same physical pages. Their
// B*G query rows per kv head (G = Hq/Hkv) are stacked into one matrix and attend to the shared
// keys once, as a dense contraction (qilem/cuda-kernel-lab, 01_decode_attention.cu:446-632 does
// the same with WMMA in two passes). Here it is a single pass with an online softmax:
//
//   S^T = K Q^T   (v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims, B = 32 dims x 16 queries)
//   O^T += V^T P^T (A = 16 dims x 32 keys, B = 32 keys x 16 queries)
//
// Computing the transposed products puts one query per lane column of every 16x16 accumulator
// (lane l holds rows 4*(l/16)+j, column l%16), so
//   * the running max / sum of a query live in the lanes of that column: a row max over a key
//     tile is an in-lane max plus two VALU lane swaps (col4_reduce), and the rescale of the output
//     accumulator by exp(m_old - m_new) is a per-lane scalar multiply;
//   * P leaves the S^T accumulator already in the B-operand layout of the PV product (the 8
//     keys a lane contributes are 4 of one 16-key tile and 4 of the next), so P needs no
//     cross-lane movement.
// K and V are staged in LDS row-major, [key][16-byte chunk], with the chunk index XOR-ed by a
// function of the key: the K A-operand reads (16 keys x one chunk per 16-lane phase) and the V
// reads below each hit every LDS bank once. The A operand of the PV product (V^T: 16 dims x 8
// keys per lane, in P's key order) comes from gfx950's transposing LDS read (ds_read_b64_tr_b16),
// two per MFMA, so V needs no transpose pass. Two LDS buffers: the global loads of block n+1 are
// in flight while block n is computed.
//
// A workgroup: 4 waves x 2 query tiles x 16 = 128 stacked query rows of one kv head, one chunk
// of prefix keys, written as the normalized partial (o, lse) of that chunk. The query rows are
// those of the sequences that share the prefix (all B, or a listed subset for one node of a
// prefix tree); chunk c of the prefix writes partial column col0 + c of each of their rows. About
// 240 VGPRs per wave and 67 KB of LDS: two such workgroups share a CU (two waves per SIMD), or one
// shares it with a decode workgroup of the fused cascade step, and the accumulators stay out of
// AGPRs, so the softmax rescale touches them in place.
#pragma once

#include <math.h>

#include <type_traits>

#include "pdattn_internal.h"
#include "timeline.h"

namespace pdattn {
namespace {

typedef _Float16 pf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 pf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 lds_f16x4;   // the builtin's type
typedef float pf32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t pu32x4 __attribute__((ext_vector_type(4)));

constexpr float kPrefixLn2 = 0.69314718055994531f;
constexpr int kPrefixWaves = 4;                               // waves per prefix workgroup
constexpr int kPrefixThreads = kPrefixWaves * 64;
constexpr int kPrefixTiles = 2;                               // 16-query tiles per wave (max)
constexpr int kPrefixRows = kPrefixWaves * kPrefixTiles * 16;  // query rows per group
constexpr int kPrefixKB = 64;                                 // keys per LDS block
constexpr int kPrefixMaxPg = 512;  // pages per chunk, i.e. chunk_tokens <= 8192

struct PSmem {
    pu32x4 K[2][kPrefixKB][16];              // [key][chunk ^ (key & 15)], 8 dims per chunk
    pu32x4 V[2][kPrefixKB][16];              // [key][chunk ^ ((key & 7) << 1)]
    int pg[kPrefixMaxPg];                    // physical pages of this chunk
    int sq[kPrefixRows];                     // sequences of this group's rows (one per G rows)
};

__device__ __forceinline__ pf32x4 mfma16x16x32(const pf16x8& a, const pf16x8& b, const pf32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Max / sum over the four lanes l, l^16, l^32, l^48 (one column of a 16x16 accumulator), left in
// all four, in the VALU: v_permlane16_swap pairs the 16-lane rows r and r^1, v_permlane32_swap the
// rows r and r^2. After a swap of a value with its own copy, result 0 holds (in every lane) the
// lower row's value and result 1 the upper row's, so the sum is formed in the same order in all
// lanes. The copy goes through an empty asm statement: given one SSA value twice, the compiler
// would treat the two results as equal and drop one.
__device__ __forceinline__ unsigned pb_opaque(unsigned v) {
    asm("" : "+v"(v));
    return v;
}
template <bool MAX>
__device__ __forceinline__ float col4_reduce(float v) {
    unsigned x = __builtin_bit_cast(unsigned, v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(x, pb_opaque(x), false, false);
    const float a = __builtin_bit_cast(float, (unsigned)r16[0]), b = __builtin_bit_cast(float, (unsigned)r16[1]);
    v = MAX ? fmaxf(a, b) : a + b;
    x = __builtin_bit_cast(unsigned, v);
    const auto r32 = __builtin_amdgcn_permlane32_swap(x, pb_opaque(x), false, false);
    const float c = __builtin_bit_cast(float, (unsigned)r32[0]), d = __builtin_bit_cast(float, (unsigned)r32[1]);
    return MAX ? fmaxf(c, d) : c + d;
}

// The work of one workgroup with NT query tiles per wave. Query tile tq of a wave is tile
// tq * PW + wave of the group's rows, so a group of up to 16 * PW * NT rows occupies the first
// NT tiles of every wave.
template <int NT>
__device__ __forceinline__ void prefix_chunk(const PrefixArgs& a, PSmem& sm, int chunk, int qgrp,
                                             int kvh) {
    constexpr int PW = kPrefixWaves, PT = kPrefixThreads, QROWS = kPrefixRows, KB = kPrefixKB;
    constexpr int SR = PT / 16;             // staging rows per pass
    constexpr int KPT = KB / SR;            // K and V rows per thread
    static_assert(KPT >= 1 && KB % SR == 0, "staging shape");
    const int G = a.Hq / a.Hkv, nq = a.ns * G;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int l16 = lane & 15, lg = lane >> 4;
    const int kbeg = chunk * a.chunk_tokens;
    const int kend = min(a.prefix_len, kbeg + a.chunk_tokens);
    const int nkeys = max(0, kend - kbeg);
    const int npg = (nkeys + kPage - 1) / kPage;
    const int nblk = (nkeys + KB - 1) / KB;
    const size_t page_bytes = (size_t)kPage * a.Hkv * 256;
    const int s0 = qgrp * (QROWS / G);                 // first member of this query group
    const int nsq = min(QROWS / G, a.ns - s0);

    // timestamps (timeline build only): 0 start, 1 page and member ids staged, 2 the first key
    // block in LDS, 3 + k key block k done (k < 24), 29 all blocks done, 30 partials written
    PD_STAMP(0);
    // page ids and member ids in one round trip
    for (int i = tid; i < npg; i += PT) sm.pg[i] = a.prefix_pages[kbeg / kPage + i];
    for (int j = tid; j < nsq; j += PT) sm.sq[j] = a.seqs ? a.seqs[s0 + j] : s0 + j;

    // Staging: thread t moves 16-byte chunk sc = t & 15 of the K and V rows sr + SR i,
    // sr = t >> 4, into [key][chunk ^ (key & 15)] (K) and [key][chunk ^ ((key & 7) << 1)] (V: the
    // swizzle under which each half-wave of the transposing reads below, 8 keys x 2 chunks x 2
    // halves, covers every LDS bank once). Keys past the chunk read the last valid key
    // instead (a real, finite row): their scores are masked to -inf below, so their weights are
    // exactly 0. The loads are cached: the other query groups of the chunk, placed on the same
    // XCD, read the same lines.
    const int sc = tid & 15, sr = tid >> 4;
    pu32x4 kst[KPT], vst[KPT];
    // A full block (64 keys, starting on a page: kbeg is a multiple of 16) holds pages
    // 4 kb .. 4 kb + 3 of the chunk: row i of this thread is slot sr of page 4 kb + i. The in-page
    // offset is therefore fixed per thread; only the page ids change from block to block.
    static_assert(KB == 4 * kPage && SR == kPage && KPT == 4, "full-block page walk");
    const uint32_t koff = (uint32_t)((sr * a.Hkv + kvh) * 256 + sc * 16);
    auto gload = [&](int kb) {
        const int key0 = kbeg + kb * KB;
        if (key0 + KB <= kend) {
#pragma unroll
            for (int i = 0; i < KPT; ++i) {
                const size_t off = (size_t)(uint32_t)sm.pg[4 * kb + i] * page_bytes + koff;
                kst[i] = *reinterpret_cast<const pu32x4*>(a.k + off);
                vst[i] = *reinterpret_cast<const pu32x4*>(a.v + off);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int key = min(key0 + sr + SR * i, kend - 1);
            const size_t off = (size_t)(uint32_t)sm.pg[(key - kbeg) >> 4] * page_bytes +
                               (size_t)(((key & 15) * a.Hkv + kvh) * 256 + sc * 16);
            kst[i] = *reinterpret_cast<const pu32x4*>(a.k + off);
            vst[i] = *reinterpret_cast<const pu32x4*>(a.v + off);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int n = sr + SR * i;
            sm.K[buf][n][sc ^ (n & 15)] = kst[i];
            sm.V[buf][n][sc ^ ((n & 7) << 1)] = vst[i];
        }
    };

    __syncthreads();   // page ids, member ids
    PD_STAMP(1);
    if (nblk > 0) gload(0);

    // B operands of S^T: Q[query][32 ks + 8 lg .. +7], query = l16 of tile tq; loaded behind the
    // first block (rows past the group read its last row and are zeroed)
    pf16x8 qb[NT][4];
    int qrow[NT];
#pragma unroll
    for (int tq = 0; tq < NT; ++tq) {
        const int r = (tq * PW + wave) * 16 + l16;    // row within the group
        const bool ok = qgrp * QROWS + r < nq;
        const int rr = ok ? r : nsq * G - 1;
        const int b = sm.sq[rr / G], g = rr % G;
        const _Float16* qp = a.q + ((size_t)b * a.Hq + kvh * G + g) * kHeadDim + 8 * lg;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qb[tq][ks] = *reinterpret_cast<const pf16x8*>(qp + 32 * ks);
        qrow[tq] = ok ? b * a.Hq + kvh * G + g : -1;
    }
    // A negative scale is moved into q: s * scale = (-s) * |scale|, and negating fp16 values
    // (their sign bits) is exact, so the loop below only ever sees a positive scale and takes the
    // maximum of the raw scores.
    const float sl2 = fabsf(a.scale_log2);
    const uint32_t qflip = a.scale_log2 < 0.f ? 0x80008000u : 0u;
#pragma unroll
    for (int tq = 0; tq < NT; ++tq)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            pu32x4 w = __builtin_bit_cast(pu32x4, qb[tq][ks]);
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = qrow[tq] < 0 ? 0u : (w[e] ^ qflip);
            qb[tq][ks] = __builtin_bit_cast(pf16x8, w);
        }

    pf32x4 acc[NT][8];
    float m_run[NT], l_run[NT];
#pragma unroll
    for (int tq = 0; tq < NT; ++tq) {
        m_run[tq] = -INFINITY;
        l_run[tq] = 0.f;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[tq][dt] = pf32x4{0.f, 0.f, 0.f, 0.f};
    }

    if (nblk > 0) lstore(0);
    __syncthreads();
    PD_STAMP(2);

    // One 64-key block. Only the chunk's last block can run past its end (EDGE): its keys past the
    // end get score -inf and weight 0, in a separate instantiation, so full blocks carry no masking.
    auto block = [&](int kb, auto EDGE) {
        constexpr bool edge = decltype(EDGE)::value;
        const int buf = kb & 1;
        const bool more = kb + 1 < nblk;
        if (more) gload(kb + 1);

        // S^T tiles: s[tq][tk][j] = score(key 16 tk + 4 lg + j, query l16 of tile tq). The K
        // fragments of key tile tk + 1 are read before the MFMAs of tile tk (the scheduling fences
        // keep them there), so the LDS latency hides under the matrix core's work.
        pf32x4 s[NT][4];
        auto kfrag = [&](int tk, pf16x8* ka) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                ka[ks] = __builtin_bit_cast(pf16x8, sm.K[buf][16 * tk + l16][(4 * ks + lg) ^ l16]);
        };
        pf16x8 ka[2][4];
        kfrag(0, ka[0]);
#pragma unroll
        for (int tk = 0; tk < 4; ++tk) {
            if (tk < 3) kfrag(tk + 1, ka[(tk + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int tq = 0; tq < NT; ++tq) {
                pf32x4 c = pf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) c = mfma16x16x32(ka[tk & 1][ks], qb[tq][ks], c);
                s[tq][tk] = c;
            }
            __builtin_amdgcn_sched_barrier(0);
        }

        // Online softmax (base 2) per query. The scores stay unscaled: the scale is positive, so
        // the maximum of the scaled scores is the scale times the maximum of the raw ones, and
        // each weight is exp2(fma(s, scale, -m)).
        const int kbase = kbeg + kb * KB + 4 * lg;
        if constexpr (edge) {
#pragma unroll
            for (int tq = 0; tq < NT; ++tq)
#pragma unroll
                for (int tk = 0; tk < 4; ++tk)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (kbase + 16 * tk + j >= kend) s[tq][tk][j] = -INFINITY;
        }
        float mn[NT];
        bool grow = false;
#pragma unroll
        for (int tq = 0; tq < NT; ++tq) {
            float mx = -INFINITY;
#pragma unroll
            for (int tk = 0; tk < 4; ++tk)
#pragma unroll
                for (int j = 0; j < 4; ++j) mx = fmaxf(mx, s[tq][tk][j]);
            mx = col4_reduce<true>(mx);
            mn[tq] = fmaxf(m_run[tq], mx * sl2);
            grow |= mn[tq] > m_run[tq];
        }
        if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
            for (int tq = 0; tq < NT; ++tq) {
                const float al = (mn[tq] > m_run[tq]) ? __builtin_amdgcn_exp2f(m_run[tq] - mn[tq]) : 1.f;
                l_run[tq] *= al;
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) acc[tq][dt] *= al;
                m_run[tq] = mn[tq];
            }
        }
        pf16x8 pb[NT][2];
#pragma unroll
        for (int tq = 0; tq < NT; ++tq) {
            const float ms = (m_run[tq] == -INFINITY) ? 0.f : m_run[tq];
#pragma unroll
            for (int tk = 0; tk < 4; ++tk)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float p = __builtin_amdgcn_exp2f(fmaf(s[tq][tk][j], sl2, -ms));
                    if constexpr (edge)   // masked keys weigh 0 whatever the scale (0 * inf would not)
                        if (kbase + 16 * tk + j >= kend) p = 0.f;
                    l_run[tq] += p;   // fp32 weights for the denominator (exact lse); PV uses
                    pb[tq][tk >> 1][(tk & 1) * 4 + j] = (_Float16)p;   // them rounded to nearest
                }
        }

        // O^T += V^T P^T. The A operand (dims 16 dt + l16, keys of k-elements 4 h .. 4 h + 3 =
        // keys 32 kb2 + 16 h + 4 lg + 0..3, the order of P's) comes from the row-major V tile by
        // transposing reads: within a 16-lane group, lane j reads 4 dims (16 dt + 4 (j & 3) ..)
        // of key 32 kb2 + 16 h + 4 lg + (j >> 2), and lane i receives element (i & 3) of lanes
        // i / 4, i / 4 + 4, ..., i.e. dim 16 dt + i of the 4 keys.
        // (the fragments of dim tile dt + 1 are read before the MFMAs of tile dt, as above)
        auto vfrag = [&](int dt, int kb2) {
            pf16x4 half[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int key = 32 * kb2 + 16 * h + 4 * lg + (l16 >> 2);
                const int chunk = 2 * dt + ((l16 & 3) >> 1);
                const _Float16* src =
                    reinterpret_cast<const _Float16*>(&sm.V[buf][key][chunk ^ ((key & 7) << 1)]) + 4 * (l16 & 1);
                half[h] = __builtin_bit_cast(pf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                    (__attribute__((address_space(3))) lds_f16x4*)(
                        (__attribute__((address_space(3))) _Float16*)src)));
            }
            return pf16x8{half[0][0], half[0][1], half[0][2], half[0][3],
                          half[1][0], half[1][1], half[1][2], half[1][3]};
        };
        pf16x8 va[2][2];
        va[0][0] = vfrag(0, 0);
        va[0][1] = vfrag(0, 1);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            if (dt < 7) {
                va[(dt + 1) & 1][0] = vfrag(dt + 1, 0);
                va[(dt + 1) & 1][1] = vfrag(dt + 1, 1);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
                for (int tq = 0; tq < NT; ++tq)
                    acc[tq][dt] = mfma16x16x32(va[dt & 1][kb2], pb[tq][kb2], acc[tq][dt]);
            __builtin_amdgcn_sched_barrier(0);
        }

        if (more) lstore(buf ^ 1);
        __syncthreads();
        if (kb < 24) PD_STAMP(3 + kb);
    };
    const int nfull = nkeys / KB;
    for (int kb = 0; kb < nfull; ++kb) block(kb, std::false_type{});
    if (nfull < nblk) block(nfull, std::true_type{});

    PD_STAMP(29);
    // normalized partial of this chunk
#pragma unroll
    for (int tq = 0; tq < NT; ++tq) {
        const float L = col4_reduce<false>(l_run[tq]);
        if (qrow[tq] < 0) continue;
        const size_t slot = (size_t)qrow[tq] * a.part_stride + a.col0 + chunk;
        const float inv = L > 0.f ? 1.f / L : 0.f;
        float* po = a.part_o + slot * kHeadDim + 4 * lg;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<pf32x4*>(po + 16 * dt) = acc[tq][dt] * inv;
        if (lg == 0)
            a.part_lse[slot] = L > 0.f ? (m_run[tq] + __builtin_amdgcn_logf(L)) * kPrefixLn2 : -INFINITY;
    }
    PD_STAMP(30);
}

// One prefix workgroup: item x of a multi-prefix launch ({page-table position of the node's
// first page, offset of its members in seqs, members, tokens, chunk tokens, first partial
// column, chunk, query group}), or chunk x / query group y of a single prefix (no item table).
__device__ __forceinline__ void prefix_workgroup(PrefixArgs a, PSmem& sm, int x, int y, int kvh) {
    int chunk = x, qgrp = y;
    if (a.items) {
        const int32_t* it = a.items + 8 * (size_t)x;
        a.prefix_pages += it[0];
        a.seqs += it[1];
        a.ns = it[2];
        a.prefix_len = it[3];
        a.chunk_tokens = it[4];
        a.col0 = it[5];
        chunk = it[6];
        qgrp = it[7];
    }
    // query tiles per wave that hold rows of this group (the same for the whole workgroup)
    const int rows = a.ns * (a.Hq / a.Hkv) - qgrp * kPrefixRows;
    if (rows > 16 * kPrefixWaves)
        prefix_chunk<kPrefixTiles>(a, sm, chunk, qgrp, kvh);
    else
        prefix_chunk<1>(a, sm, chunk, qgrp, kvh);
}

}  // namespace
}  // namespace pdattn
