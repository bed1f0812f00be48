// cascade.hip -- the prefix kernels of the shared-prefix (cascade) path: one workgroup per
// (prefix chunk or tree item, query group, kv head). The 4-wave body (prefix_body.h) serves tree
// items and prefixes with up to 128 rows per kv head; a single prefix with more rows runs on the
// 8-wave key-split body below.
#include "timeline.h"

PD_TIMELINE_TABLE(prefix)

#include "prefix_body.h"

namespace pdattn {
namespace {

// Two workgroups per CU (two waves per SIMD): one wave's softmax runs while the other's MFMAs
// occupy the matrix core.
__global__ __launch_bounds__(kPrefixThreads, 2) void cascade_prefix_kernel(PrefixArgs a) {
    __shared__ PSmem sm;
    prefix_workgroup(a, sm, blockIdx.x, blockIdx.y, blockIdx.z);
}

// ---------------------------------------------------------------------------------------------
// The key-split body: 8 waves over 128 stacked query rows of one kv head and one chunk, one
// workgroup per CU.
//
// Waves 0-3 (group 0) take the chunk's first ceil(nblk / 2) 64-key blocks and waves 4-7 (group 1)
// the rest; wave w and wave w + 4 hold the same 32 query rows, and each SIMD holds one wave of each
// group. A step of a wave is an MFMA phase (the PV product of block i - 1, then the scores of block
// i) and a VALU phase (the online softmax of a block); group 0 runs them in that order, group 1 the
// other way round (the softmax of block i - 1 first), so each step starts with one wave's MFMAs
// beside the other's VALU work on every SIMD. One workgroup barrier per step. At the end wave
// w + 4 hands its (maximum, sum, accumulators) to wave w through LDS, and wave w writes the
// chunk's partial: one partial per row for the 2 x 256 keys of a 512-token chunk, half the partial
// bytes that 256-row workgroups over 256-token chunks write for the same work per workgroup.
//
// Each group stages its own blocks, K and V, into two LDS buffers each, by direct global->LDS
// loads (global_load_lds_dwordx4: no registers, no LDS store instructions). Block i's K is read
// by the scores in step i and its V by the PV product in step i + 1, so after the barrier that
// starts step i a wave issues K of block i + 1 and V of block i (their buffers' last readers ran
// in step i - 1) and waits for them at the end of the step.
constexpr int kKSWaves = 8;
constexpr int kKSThreads = kKSWaves * 64;
constexpr int kKSRows = 4 * kPrefixTiles * 16;   // 128 query rows per workgroup

struct KSSmem {
    pu32x4 K[2][2][kPrefixKB][16];   // [group][buffer][key][chunk ^ (key & 15)]
    pu32x4 V[2][2][kPrefixKB][16];   // [group][buffer][key][chunk ^ ((key & 7) << 1)]
    float ml[4][kPrefixTiles][2][64];   // group 1's maximum and sum per wave, tile and lane
    int pg[kPrefixMaxPg];
};

// LDS writes done, then the workgroup barrier. The staging loads stay in flight across it (a
// __syncthreads() fence would wait for them); the memory clobber keeps the compiler's LDS
// accesses on their side of it, the scheduling fences every other instruction.
__device__ __forceinline__ void ks_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// 16 bytes per lane from global memory into LDS: lane i's bytes land at lds + 16 i (M0 holds the
// LDS address; one wait state between the M0 write and the load). The compiler does not count
// these loads: the waits below are explicit. M0 is a reserved register to the compiler (hipcc
// warns that a clobber of it is not preserved); on gfx950 nothing else in these kernels reads or
// writes it, which the build lint checks on the assembly.
__device__ __forceinline__ void ks_dma(const uint8_t* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(lds) : "memory", "m0");
}
// the same from a wave-uniform base (scalar registers) plus a 32-bit per-lane offset
__device__ __forceinline__ void ks_dma_s(const uint8_t* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :: "v"(off), "s"(base), "s"(lds) : "memory", "m0");
}
// Wait until at most n (0, 4 or 8, wave-uniform) of this wave's loads are in flight.
__device__ __forceinline__ void ks_wait_loads(int n) {
    if (n >= 8)
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (n >= 4)
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// The value itself, as a new value in every call (volatile: not hoisted out of a loop, not merged
// with another call's).
__device__ __forceinline__ uint32_t ks_fresh(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

template <int NT>
__device__ __forceinline__ void prefix_chunk_ks(const PrefixArgs& a, KSSmem& sm, int chunk, int qgrp,
                                                int kvh) {
    constexpr int QROWS = kKSRows, KB = kPrefixKB, PT = kKSThreads;
    const int G = a.Hq / a.Hkv, nq = a.ns * G;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int grp = wave >> 2, w4 = wave & 3;
    const int l16 = lane & 15, lg = lane >> 4;
    const int kbeg = chunk * a.chunk_tokens;
    const int kend = min(a.prefix_len, kbeg + a.chunk_tokens);
    const int nkeys = max(0, kend - kbeg);
    const int npg = (nkeys + kPage - 1) / kPage;
    const int nblk = (nkeys + KB - 1) / KB;
    const int nsteps = (nblk + 1) / 2;                        // group 0's blocks
    const int g0 = grp == 0 ? kbeg : min(kend, kbeg + nsteps * KB);   // this group's keys [g0, g1)
    const int g1 = grp == 0 ? min(kend, kbeg + nsteps * KB) : kend;
    const int nbg = (g1 - g0 + KB - 1) / KB;                  // this group's blocks
    const int nfg = (g1 - g0) / KB;                           // of them full
    const int pg0 = (g0 - kbeg) / kPage;                      // its first page within the chunk
    const size_t page_bytes = (size_t)kPage * a.Hkv * 256;

    // timestamps (timeline build only), as in prefix_chunk, seen by wave 0 (group 0)
    PD_STAMP(0);
    for (int i = tid; i < npg; i += PT) sm.pg[i] = a.prefix_pages[kbeg / kPage + i];

    // Staging: wave w4 of a group moves rows 16 w4 + 4 i + (lane >> 4) (i < 4) of each of the
    // group's blocks, lane & 15 being the 16-byte position in the LDS row; position p of row n holds
    // chunk p ^ (n & 15) of K and p ^ ((n & 7) << 1) of V (the swizzles of prefix_chunk). In a full
    // block these rows are slots 4 i + (lane >> 4) of the block's page w4.
    static_assert(KB == 4 * kPage, "full-block page walk");
    const uint32_t lds_k = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)&sm.K[grp][0][16 * w4][0];
    const uint32_t lds_v = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)&sm.V[grp][0][16 * w4][0];
    constexpr uint32_t kBufBytes = KB * 16 * 16;
    auto dma = [&](int j, bool is_v) {
        const uint8_t* base = is_v ? a.v : a.k;
        const uint32_t dst = (is_v ? lds_v : lds_k) + (uint32_t)(j & 1) * kBufBytes;
        const int key0 = g0 + j * KB;
        if (key0 + KB <= g1) {
            const uint8_t* pb = base + (size_t)(uint32_t)__builtin_amdgcn_readfirstlane(sm.pg[pg0 + 4 * j + w4]) * page_bytes;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n = 4 * i + (lane >> 4);
                const int ch = (lane & 15) ^ (is_v ? (n & 7) << 1 : n);
                ks_dma_s(pb, (uint32_t)((n * a.Hkv + kvh) * 256 + ch * 16), dst + 1024 * i);
            }
            return;
        }
        // the partial last block: rows past the group's keys read its last key (finite; weight 0)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = 4 * i + (lane >> 4);
            const int key = min(key0 + 16 * w4 + n, g1 - 1);
            const int ch = (lane & 15) ^ (is_v ? (n & 7) << 1 : n);
            ks_dma(base + (size_t)(uint32_t)sm.pg[(key - kbeg) >> 4] * page_bytes +
                       (((key & 15) * a.Hkv + kvh) * 256 + ch * 16),
                   dst + 1024 * i);
        }
    };

    // Prologue: group 0's waves start the K rows of their first block from a page id read straight
    // from the page table (a full first block), then every wave loads its q rows while the page
    // ids reach LDS.
    bool k0 = false;
    if (grp == 0 && g0 + KB <= g1) {
        const uint8_t* pb = a.k + (size_t)(uint32_t)__builtin_amdgcn_readfirstlane(
                                      a.prefix_pages[kbeg / kPage + w4]) * page_bytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = 4 * i + (lane >> 4);
            ks_dma_s(pb, (uint32_t)((n * a.Hkv + kvh) * 256 + (((lane & 15) ^ n) * 16)), lds_k + 1024 * i);
        }
        k0 = true;
    }

    // B operands of S^T, as in prefix_chunk; tile tq of wave w (and of wave w + 4) is tile
    // tq * 4 + w of the workgroup's rows, row r being head kvh * G + r % G of sequence r / G (a
    // single prefix: the rows of sequences 0 .. ns - 1)
    pf16x8 qb[NT][4];
    int qrow[NT];
#pragma unroll
    for (int tq = 0; tq < NT; ++tq) {
        const int r = qgrp * QROWS + (tq * 4 + w4) * 16 + l16;
        const bool ok = r < nq;
        const int rr = ok ? r : nq - 1;
        const _Float16* qp = a.q + ((size_t)(rr / G) * a.Hq + kvh * G + rr % G) * kHeadDim + 8 * lg;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qb[tq][ks] = *reinterpret_cast<const pf16x8*>(qp + 32 * ks);
        qrow[tq] = ok ? (rr / G) * a.Hq + kvh * G + rr % G : -1;
    }
    __syncthreads();   // page ids
    PD_STAMP(1);
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

    // K of block 0 in LDS before the first step (group 0's full first block landed with the q rows)
    if (nbg > 0 && !k0) dma(0, false);
    ks_wait_loads(0);
    ks_barrier();
    PD_STAMP(2);

    // The scores of a block between its MFMA and VALU phases; then, in s[tq][0..1], its fp16
    // weights until the next MFMA phase (one set of registers carried across the phases).
    pf32x4 s[NT][4];

    // LDS byte addresses of the fragment reads, formed in each phase from a per-lane base (held
    // opaque there, so the compiler does not keep every fragment's address live across the loop).
    // K: key 16 tk + l16, chunk (4 ks + lg) ^ l16 = bits 6-7 ks ^ (l16 >> 2), bits 4-5 lg ^ (l16 & 3):
    // base ^ (ks << 6), + 4096 tk. V (transposing reads): key 32 kb2 + 16 h + kl, kl = 4 lg + l16 / 4,
    // chunk (2 dt + c0) ^ sw, sw = (kl & 7) << 1, c0 = (l16 & 3) >> 1, plus 8 bytes for odd l16:
    // base ^ (dt << 5), + 256 (32 kb2 + 16 h). The arrays and buffers start at multiples of 256
    // bytes, so the XOR-ed bits of a base are its swizzle bits alone.
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    lds_u8* const lds = (lds_u8*)(&sm);
    const uint32_t k_lane = (uint32_t)((uintptr_t)&sm.K[grp][0][0][0] - (uintptr_t)&sm) + l16 * 256 +
                            ((((l16 >> 2) << 2) | (lg ^ (l16 & 3))) << 4);
    const int kl = 4 * lg + (l16 >> 2);
    const uint32_t v_lane = (uint32_t)((uintptr_t)&sm.V[grp][0][0][0] - (uintptr_t)&sm) + kl * 256 +
                            ((((kl & 7) << 1) | ((l16 & 3) >> 1)) << 4) + 8 * (l16 & 1);

    // The PV product of block j (O^T += V^T P^T, the weights in s[tq][0..1]).
    auto pv = [&](int j) {
        const uint32_t vb = ks_fresh(v_lane) + (uint32_t)(j & 1) * kBufBytes;
        auto vfrag = [&](int dt, int kb2) {
            const uint32_t ad = vb ^ (uint32_t)(dt << 5);
            pf16x4 half[2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
                half[h] = __builtin_bit_cast(pf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                    (__attribute__((address_space(3))) lds_f16x4*)(lds + ad + 256 * (32 * kb2 + 16 * h))));
            return pf16x8{half[0][0], half[0][1], half[0][2], half[0][3],
                          half[1][0], half[1][1], half[1][2], half[1][3]};
        };
        // one register set, refilled operand by operand: the fragment of (dt + 1, kb2) is read
        // right after the MFMAs of (dt, kb2), eight MFMAs before its own
        pf16x8 va[2];
        va[0] = vfrag(0, 0);
        va[1] = vfrag(0, 1);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
                for (int tq = 0; tq < NT; ++tq)
                    acc[tq][dt] = mfma16x16x32(va[kb2], __builtin_bit_cast(pf16x8, s[tq][kb2]), acc[tq][dt]);
                if (dt < 7) va[kb2] = vfrag(dt + 1, kb2);
                __builtin_amdgcn_sched_barrier(0);
            }
    };
    // The scores of block m (S^T = K Q^T) into s.
    auto qk = [&](int m) {
        const uint32_t kb = ks_fresh(k_lane) + (uint32_t)(m & 1) * kBufBytes;
        auto kfrag = [&](int tk, int ks) {
            return __builtin_bit_cast(pf16x8, *(const __attribute__((address_space(3))) pu32x4*)(
                                                  lds + ((kb ^ (uint32_t)(ks << 6)) + 4096 * tk)));
        };
        // one register set, refilled as in pv
        pf16x8 ka[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) ka[ks] = kfrag(0, ks);
#pragma unroll
        for (int tk = 0; tk < 4; ++tk) {
            pf32x4 c[NT];
#pragma unroll
            for (int tq = 0; tq < NT; ++tq) c[tq] = pf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
                for (int tq = 0; tq < NT; ++tq) c[tq] = mfma16x16x32(ka[ks], qb[tq][ks], c[tq]);
                if (tk < 3) ka[ks] = kfrag(tk + 1, ks);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int tq = 0; tq < NT; ++tq) s[tq][tk] = c[tq];
        }
    };

    // VALU phase, softmax of block m of the group (EDGE: the chunk's partial last block, keys past
    // its end weigh 0), the steps of prefix_chunk's.
    auto softmax = [&](int m, auto EDGE) {
        constexpr bool edge = decltype(EDGE)::value;
        const int kbase = g0 + m * KB + 4 * lg;
        if constexpr (edge) {
#pragma unroll
            for (int tq = 0; tq < NT; ++tq)
#pragma unroll
                for (int tk = 0; tk < 4; ++tk)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (kbase + 16 * tk + j >= g1) s[tq][tk][j] = -INFINITY;
        }
        // The rescale runs in every block (by 1 where no maximum grew, which changes nothing): a
        // branch around it makes the register allocator copy the accumulators at the merge.
#pragma unroll
        for (int tq = 0; tq < NT; ++tq) {
            float mx = -INFINITY;
#pragma unroll
            for (int tk = 0; tk < 4; ++tk)
#pragma unroll
                for (int j = 0; j < 4; ++j) mx = fmaxf(mx, s[tq][tk][j]);
            mx = col4_reduce<true>(mx);
            const float mn = fmaxf(m_run[tq], mx * sl2);
            const float al = (mn > m_run[tq]) ? __builtin_amdgcn_exp2f(m_run[tq] - mn) : 1.f;
            l_run[tq] *= al;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) acc[tq][dt] *= al;
            m_run[tq] = mn;
        }
#pragma unroll
        for (int tq = 0; tq < NT; ++tq) {
            const float ms = (m_run[tq] == -INFINITY) ? 0.f : m_run[tq];
            pf16x8 pb[2];
#pragma unroll
            for (int tk = 0; tk < 4; ++tk)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float p = __builtin_amdgcn_exp2f(fmaf(s[tq][tk][j], sl2, -ms));
                    if constexpr (edge)   // masked keys weigh 0 whatever the scale (0 * inf would not)
                        if (kbase + 16 * tk + j >= g1) p = 0.f;
                    l_run[tq] += p;
                    pb[tk >> 1][(tk & 1) * 4 + j] = (_Float16)p;
                }
            s[tq][0] = __builtin_bit_cast(pf32x4, pb[0]);
            s[tq][1] = __builtin_bit_cast(pf32x4, pb[1]);
        }
    };
    // The VALU phase sets each step's pace (a lone wave issues VALU work at about half the SIMD's
    // rate), so the wave in it takes issue priority over its SIMD partner in the MFMA phase.
    auto valu_phase = [&](int m) {
        __builtin_amdgcn_s_setprio(2);
        if (m < nfg)
            softmax(m, std::false_type{});
        else
            softmax(m, std::true_type{});
        __builtin_amdgcn_s_setprio(0);
    };
    // Block loads of step i, issued after the barrier that starts it: K of block i + 1 (its buffer's
    // last reader, the scores of block i - 1, ran in step i - 1) and V of block i (the PV product of
    // block i - 2 ran in step i - 1); waited for at the end of the step, before the barrier that
    // starts step i + 1, where they are read.
    auto issue = [&](int i) {
        if (i + 1 < nbg) dma(i + 1, false);
        if (i < nbg) dma(i, true);
    };

    // The steps, one loop per group (each straight-line), one barrier per step. Group 0, step i:
    // MFMA phase (pv(i - 1), qk(i)), then VALU phase (softmax of block i). Group 1: VALU phase
    // (softmax of block i - 1), then MFMA phase (pv(i - 1), qk(i)). On each SIMD one wave of each
    // group, so a step starts with one wave's MFMAs beside the other's VALU work, and from there
    // the two waves overlap as their phases allow.
    if (grp == 0) {
        for (int i = 0; i <= nsteps; ++i) {
            issue(i);
            if (i >= 1) pv(i - 1);
            if (i < nbg) qk(i);
            if (i >= 1 && i - 1 < 24) PD_STAMP(3 + i - 1);
            if (i < nsteps) valu_phase(i);
            ks_wait_loads(0);
            ks_barrier();
        }
    } else {
        for (int i = 0; i <= nsteps; ++i) {
            issue(i);
            if (i >= 1 && i - 1 < nbg) {
                valu_phase(i - 1);
                pv(i - 1);
            }
            if (i < nbg) qk(i);
            ks_wait_loads(0);
            ks_barrier();
        }
    }
    PD_STAMP(29);

    // Group 1's state through LDS (the K buffers are no longer read: every score product was done
    // before the last barrier), then group 0 combines the two key ranges and writes the partial.
    float* xacc = reinterpret_cast<float*>(&sm.K[0][0][0][0]);   // [w4][tq][dt][lane][4]
    if (grp == 1) {
#pragma unroll
        for (int tq = 0; tq < NT; ++tq) {
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
                *reinterpret_cast<pf32x4*>(xacc + (((w4 * NT + tq) * 8 + dt) * 64 + lane) * 4) = acc[tq][dt];
            sm.ml[w4][tq][0][lane] = m_run[tq];
            sm.ml[w4][tq][1][lane] = l_run[tq];
        }
    }
    __syncthreads();
    if (grp == 1) return;
#pragma unroll
    for (int tq = 0; tq < NT; ++tq) {
        const float m1 = sm.ml[w4][tq][0][lane], l1 = sm.ml[w4][tq][1][lane];
        const float m = fmaxf(m_run[tq], m1);
        const float a0 = m_run[tq] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[tq] - m);
        const float a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
        l_run[tq] = l_run[tq] * a0 + l1 * a1;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const pf32x4 o1 = *reinterpret_cast<const pf32x4*>(xacc + (((w4 * NT + tq) * 8 + dt) * 64 + lane) * 4);
            acc[tq][dt] = acc[tq][dt] * a0 + o1 * a1;
        }
        m_run[tq] = m;
    }
    // (the output fields are read again from the kernarg segment, and a row's validity is tested
    // again, rather than held in scalar registers across the loops)
    typedef const __attribute__((address_space(4))) PrefixArgs* ArgPtr;
    ArgPtr ka = (ArgPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ka));
#pragma unroll
    for (int tq = 0; tq < NT; ++tq) {
        const float L = col4_reduce<false>(l_run[tq]);
        const int qr = (int)ks_fresh((uint32_t)qrow[tq]);
        if (qr < 0) continue;
        const size_t slot = (size_t)qr * ka->part_stride + ka->col0 + chunk;
        const float inv = L > 0.f ? 1.f / L : 0.f;
        float* po = ka->part_o + slot * kHeadDim + 4 * lg;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<pf32x4*>(po + 16 * dt) = acc[tq][dt] * inv;
        if (lg == 0)
            ka->part_lse[slot] = L > 0.f ? (m_run[tq] + __builtin_amdgcn_logf(L)) * kPrefixLn2 : -INFINITY;
    }
    PD_STAMP(30);
}

// One workgroup per CU: 8 waves of at most 256 VGPRs fill each SIMD's registers, and the four
// key buffers take 134 KB of LDS. Workgroup (x, y) = (query group * Hkv + kv head, chunk):
// workgroups go to the XCDs round robin, so with Hkv a multiple of 8 every chunk of a (query group,
// kv head) runs on one XCD, whose L2 then holds whole stretches of each row's partials (a row's
// chunks are adjacent in memory) when they are written back.
__global__ __launch_bounds__(kKSThreads, 1) void cascade_prefix_ks_kernel(PrefixArgs a) {
    __shared__ KSSmem sm;
    const int qgrp = blockIdx.x / a.Hkv, kvh = blockIdx.x % a.Hkv;
    const int rows = a.ns * (a.Hq / a.Hkv) - qgrp * kKSRows;
    if (rows > 16 * 4)
        prefix_chunk_ks<kPrefixTiles>(a, sm, blockIdx.y, qgrp, kvh);
    else
        prefix_chunk_ks<1>(a, sm, blockIdx.y, qgrp, kvh);
}

}  // namespace

int prefix_rows_per_workgroup() { return kPrefixRows; }

hipError_t launch_cascade_prefix(const PrefixArgs& a, int G, hipStream_t s) {
    if (a.Hkv <= 0) return hipSuccess;
    if (a.items) {
        // num_chunks = number of items
        if (a.num_chunks <= 0) return hipSuccess;
        cascade_prefix_kernel<<<dim3(a.num_chunks, 1, a.Hkv), kPrefixThreads, 0, s>>>(a);
        return hipGetLastError();
    }
    const int rows = a.ns * G;
    if (a.num_chunks <= 0 || rows <= 0) return hipSuccess;
    if (rows > kPrefixRows && !a.seqs) {
        dim3 grid((rows + kKSRows - 1) / kKSRows * a.Hkv, a.num_chunks);
        cascade_prefix_ks_kernel<<<grid, kKSThreads, 0, s>>>(a);
        return hipGetLastError();
    }
    dim3 grid(a.num_chunks, (rows + kPrefixRows - 1) / kPrefixRows, a.Hkv);
    cascade_prefix_kernel<<<grid, kPrefixThreads, 0, s>>>(a);
    return hipGetLastError();
}

int occupancy_cascade_prefix(int G) {
    (void)G;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&cascade_prefix_kernel), kPrefixThreads, 0) != hipSuccess)
        return 1;
    return n > 0 ? n : 1;
}

}  // namespace pdattn
