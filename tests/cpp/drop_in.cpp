// drop_in.cpp -- the reference's decode-attention call sequence, in C++, through libpdattn's C ABI.
//
// qilem/cuda-kernel-lab's experiment 01 checks itself from main(): its correctness cases
// (01_decode_attention.cu:749-781) run decode_attention with the three split settings
// {no split, heuristic, 7 chunks} (01:763), and its cascade cases (01:782-815) run
// shared_prefix_pages / plan_cascade / cascade_decode on shared-prefix batches, including a batch
// without sharing (01:810-815). This program makes the same calls through include/pdattn.h, the
// way a C++ caller of the reference would after switching, plus the plan / run path, and checks
// every result against the fp64 CPU oracle (oracle/pdattn_oracle.c, test infrastructure) with
// the parity bar: max |out - ref| <= 2e-3, |lse - ref| <= 1e-4 + 1e-4 |ref|, -inf where the
// oracle has -inf. Batches follow 01:333-368 and 01:714-742: page counts ceil(L / 16), a shuffled
// permutation of physical pages (std::mt19937), q / K / V uniform in (-1, 1) rounded to fp16.
//
// pdattn_drop_in_checks() returns the number of failed cases. Built twice (tests/cpp/Makefile):
// as libdrop_in.so, which tests/test_cpp_drop_in_gpu.py calls in its own process, and with
// DROP_IN_MAIN as the standalone program drop_in (exit status 0 when every case passes).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <random>
#include <string>
#include <vector>

#include "pdattn.h"

extern "C" {
void oracle_decode_mt(const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* indptr,
                      const int32_t* indices, const int32_t* last, int B, int Hq, int Hkv, int kv_start,
                      double sm_scale, double* out, double* lse, int threads);
double oracle_half_to_double(uint16_t h);
uint16_t oracle_double_to_half(double x);
int oracle_shared_prefix_pages(const int32_t* indptr, const int32_t* indices, int B);
}

namespace {

constexpr int kD = 128, kPage = 16;
int g_failures = 0;

#define HIP_OK(call)                                                                              \
    do {                                                                                          \
        hipError_t e_ = (call);                                                                   \
        if (e_ != hipSuccess) {                                                                   \
            std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #call, hipGetErrorString(e_)); \
            std::exit(2);                                                                         \
        }                                                                                         \
    } while (0)
#define PD_OK(call)                                                                               \
    do {                                                                                          \
        int s_ = (call);                                                                          \
        if (s_ != PDATTN_OK) {                                                                    \
            std::fprintf(stderr, "%s:%d %s: %s (%s)\n", __FILE__, __LINE__, #call,                \
                         pdattn_strerror(s_), pdattn_last_error());                              \
            std::exit(2);                                                                         \
        }                                                                                         \
    } while (0)

// A batch on the host: CSR page table, fp16 bits of q [B,Hq,128] and K/V [pages,16,Hkv,128].
struct Batch {
    int B = 0, Hq = 0, Hkv = 0, pages = 0;
    std::vector<int32_t> lens, indptr, indices, last;
    std::vector<uint16_t> q, k, v;
};

void fill_uniform(std::vector<uint16_t>& x, size_t n, std::mt19937& rng) {
    std::uniform_real_distribution<float> u(-1.f, 1.f);
    x.resize(n);
    for (auto& e : x) e = oracle_double_to_half(u(rng));
}

// Sequences of the given lengths, each on its own pages, physical pages shuffled.
Batch make_batch(const std::vector<int>& lens, int Hq, int Hkv, unsigned seed) {
    Batch b;
    b.B = (int)lens.size();
    b.Hq = Hq;
    b.Hkv = Hkv;
    b.lens.assign(lens.begin(), lens.end());
    b.indptr.assign(b.B + 1, 0);
    for (int i = 0; i < b.B; ++i) {
        const int np = (lens[i] + kPage - 1) / kPage;
        b.indptr[i + 1] = b.indptr[i] + np;
        b.last.push_back(np ? lens[i] - (np - 1) * kPage : 0);
    }
    b.pages = b.indptr[b.B];
    std::mt19937 rng(seed);
    b.indices.resize(b.pages);
    std::iota(b.indices.begin(), b.indices.end(), 0);
    std::shuffle(b.indices.begin(), b.indices.end(), rng);
    fill_uniform(b.q, (size_t)b.B * Hq * kD, rng);
    fill_uniform(b.k, (size_t)std::max(1, b.pages) * kPage * Hkv * kD, rng);
    fill_uniform(b.v, (size_t)std::max(1, b.pages) * kPage * Hkv * kD, rng);
    return b;
}

// Every sequence starts with the same lp / 16 physical pages, then has `suffix[i]` tokens on
// pages of its own (make_shared_prefix_batch, 01:714-742).
Batch make_shared_prefix_batch(int lp, const std::vector<int>& suffix, int Hq, int Hkv, unsigned seed) {
    Batch b;
    b.B = (int)suffix.size();
    b.Hq = Hq;
    b.Hkv = Hkv;
    const int pp = lp / kPage;
    int own = 0;
    for (int s : suffix) own += (s + kPage - 1) / kPage;
    b.pages = pp + own;
    std::mt19937 rng(seed);
    std::vector<int32_t> perm(b.pages);
    std::iota(perm.begin(), perm.end(), 0);
    std::shuffle(perm.begin(), perm.end(), rng);
    int next = pp;
    b.indptr.assign(b.B + 1, 0);
    for (int i = 0; i < b.B; ++i) {
        const int np_own = (suffix[i] + kPage - 1) / kPage;
        for (int p = 0; p < pp; ++p) b.indices.push_back(perm[p]);
        for (int p = 0; p < np_own; ++p) b.indices.push_back(perm[next++]);
        b.indptr[i + 1] = (int32_t)b.indices.size();
        b.lens.push_back(lp + suffix[i]);
        b.last.push_back(suffix[i] - (np_own - 1) * kPage);
    }
    fill_uniform(b.q, (size_t)b.B * Hq * kD, rng);
    fill_uniform(b.k, (size_t)b.pages * kPage * Hkv * kD, rng);
    fill_uniform(b.v, (size_t)b.pages * kPage * Hkv * kD, rng);
    return b;
}

template <class T>
T* upload(const std::vector<T>& h) {
    T* d = nullptr;
    HIP_OK(hipMalloc(&d, std::max<size_t>(sizeof(T), sizeof(T) * h.size())));
    if (!h.empty()) HIP_OK(hipMemcpy(d, h.data(), sizeof(T) * h.size(), hipMemcpyHostToDevice));
    return d;
}

// Device copies of a batch and its outputs.
struct DeviceBatch {
    uint16_t *q = nullptr, *k = nullptr, *v = nullptr, *out = nullptr;
    int32_t *indptr = nullptr, *indices = nullptr, *last = nullptr;
    float* lse = nullptr;
    size_t rows = 0;
    explicit DeviceBatch(const Batch& b) {
        q = upload(b.q);
        k = upload(b.k);
        v = upload(b.v);
        indptr = upload(b.indptr);
        indices = upload(b.indices);
        last = upload(b.last);
        rows = (size_t)b.B * b.Hq;
        HIP_OK(hipMalloc(&out, sizeof(uint16_t) * std::max<size_t>(1, rows) * kD));
        HIP_OK(hipMalloc(&lse, sizeof(float) * std::max<size_t>(1, rows)));
    }
    ~DeviceBatch() {
        for (void* p : {(void*)q, (void*)k, (void*)v, (void*)out, (void*)indptr, (void*)indices,
                        (void*)last, (void*)lse})
            (void)hipFree(p);
    }
    // the launch block of decode_attention (DecodeParams, 01:51-65)
    pdattn_decode_params params(const Batch& b, int num_chunks, int chunk_tokens) const {
        pdattn_decode_params p{};
        p.q = q;
        p.k_cache = k;
        p.v_cache = v;
        p.kv_indptr = indptr;
        p.kv_indices = indices;
        p.kv_last_page_len = last;
        p.B = b.B;
        p.Hq = b.Hq;
        p.Hkv = b.Hkv;
        p.num_chunks = num_chunks;
        p.chunk_tokens = chunk_tokens;
        p.kv_start = 0;
        p.chunk_base = 0;
        p.part_stride = num_chunks;
        p.sm_scale = 1.0f / std::sqrt((float)kD);
        return p;
    }
};

// The parity bar against the fp64 oracle; prints one line per case.
void check(const char* tag, const Batch& b, const DeviceBatch& db) {
    HIP_OK(hipDeviceSynchronize());
    const size_t rows = db.rows;
    std::vector<uint16_t> out(rows * kD);
    std::vector<float> lse(rows);
    if (rows) {
        HIP_OK(hipMemcpy(out.data(), db.out, sizeof(uint16_t) * out.size(), hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(lse.data(), db.lse, sizeof(float) * lse.size(), hipMemcpyDeviceToHost));
    }
    std::vector<double> ro(rows * kD), rl(rows);
    oracle_decode_mt(b.q.data(), b.k.data(), b.v.data(), b.indptr.data(),
                     b.indices.empty() ? nullptr : b.indices.data(), b.last.data(), b.B, b.Hq, b.Hkv,
                     0, 1.0 / std::sqrt((double)kD), ro.data(), rl.data(), 8);
    double emax = 0.0, lmax = 0.0;
    bool ok = true;
    for (size_t i = 0; i < out.size(); ++i) {
        const double g = oracle_half_to_double(out[i]);
        if (!std::isfinite(g)) ok = false;
        emax = std::max(emax, std::fabs(g - ro[i]));
    }
    for (size_t i = 0; i < rows; ++i) {
        if (std::isinf(rl[i]) && rl[i] < 0) {
            if (!(std::isinf(lse[i]) && lse[i] < 0)) ok = false;
            continue;
        }
        const double err = std::fabs((double)lse[i] - rl[i]);
        lmax = std::max(lmax, err);
        if (!(err <= 1e-4 + 1e-4 * std::fabs(rl[i]))) ok = false;
    }
    ok = ok && emax <= 2e-3;
    std::printf("%-52s out max_abs %.3e  lse max_abs %.3e  %s\n", tag, emax, lmax, ok ? "PASS" : "FAIL");
    if (!ok) ++g_failures;
}

// decode_attention with the reference's three split settings, and plan / run.
void decode_case(const char* name, const std::vector<int>& lens, int Hq, int Hkv, unsigned seed) {
    const Batch b = make_batch(lens, Hq, Hkv, seed);
    DeviceBatch db(b);
    const int G = Hq / Hkv;
    const int max_len = *std::max_element(lens.begin(), lens.end());
    char tag[160];
    // a caller that takes page tables from elsewhere checks them first: this one is valid, and
    // the same table with one page id past the cache is refused
    PD_OK(pdattn_check_page_table(b.indptr.data(), b.indices.data(), b.last.data(), b.B, b.pages));
    if (b.pages > 0) {
        std::vector<int32_t> bad = b.indices;
        bad[bad.size() / 2] = b.pages;
        const int st = pdattn_check_page_table(b.indptr.data(), bad.data(), b.last.data(), b.B, b.pages);
        std::printf("%-52s %s\n", (std::string(name) + " page id past the cache refused").c_str(),
                    st == PDATTN_ERR_PAGE_TABLE ? "PASS" : "FAIL");
        if (st != PDATTN_ERR_PAGE_TABLE) ++g_failures;
    }
    for (int force : {1, 0, 7}) {
        int nc = 0, ct = 0;
        PD_OK(pdattn_plan_chunks(G, 2, b.B, Hkv, max_len, force, &nc, &ct));
        pdattn_decode_params p = db.params(b, nc, ct);
        pdattn_workspace ws{};
        PD_OK(pdattn_decode_attention(&p, G, 2, db.out, db.lse, &ws, nullptr));
        std::snprintf(tag, sizeof tag, "%s decode_attention chunks=%d", name, nc);
        check(tag, b, db);
        pdattn_workspace_release(&ws);
        // the same call for a caller that cannot allocate (partials in the library's own array)
        if (pdattn_decode_workspace_size(b.B, Hq, nc) <= PDATTN_NOALLOC_SCRATCH_BYTES) {
            PD_OK(pdattn_decode_attention_noalloc(&p, G, 2, db.out, db.lse, nullptr));
            std::snprintf(tag, sizeof tag, "%s decode_attention_noalloc chunks=%d", name, nc);
            check(tag, b, db);
        }
        // the same arguments, the pages cut into equal ranges on the device, in a workspace the
        // caller sized with pdattn_decode_balanced_workspace_size
        const size_t bb = pdattn_decode_balanced_workspace_size(&p, G);
        void* wb = nullptr;
        HIP_OK(hipMalloc(&wb, bb > 0 ? bb : 256));
        pdattn_workspace wsb{wb, bb, 0};
        PD_OK(pdattn_decode_attention_balanced(&p, G, 2, db.out, db.lse, &wsb, nullptr));
        std::snprintf(tag, sizeof tag, "%s decode_attention_balanced chunks=%d", name, nc);
        check(tag, b, db);
        HIP_OK(hipFree(wb));
    }
    pdattn_plan* plan = nullptr;
    PD_OK(pdattn_plan_create(b.indptr.data(), b.last.data(), b.B, Hq, Hkv, 0, 0, &plan));
    const size_t bytes = pdattn_plan_workspace_size(plan);
    void* ws = nullptr;
    HIP_OK(hipMalloc(&ws, bytes));
    PD_OK(pdattn_plan_upload(plan, ws, bytes, nullptr));
    PD_OK(pdattn_plan_run(plan, db.q, db.k, db.v, db.indptr, db.indices, db.last,
                          1.0f / std::sqrt((float)kD), db.out, db.lse, ws, bytes, nullptr));
    std::snprintf(tag, sizeof tag, "%s plan/run", name);
    check(tag, b, db);
    pdattn_plan_destroy(plan);
    HIP_OK(hipFree(ws));
}

// shared_prefix_pages, plan_cascade and cascade_decode on a shared-prefix batch.
void cascade_case(const char* name, int lp, const std::vector<int>& suffix, int Hq, int Hkv,
                  unsigned seed) {
    const Batch b = make_shared_prefix_batch(lp, suffix, Hq, Hkv, seed);
    DeviceBatch db(b);
    const int pp = pdattn_shared_prefix_pages(b.indptr.data(), b.indices.data(), b.B);
    const int pref = oracle_shared_prefix_pages(b.indptr.data(), b.indices.data(), b.B);
    if (pp != lp / kPage || pp != pref) {
        std::printf("%s shared_prefix_pages %d (oracle %d, expected %d)  FAIL\n", name, pp, pref, lp / kPage);
        ++g_failures;
    }
    pdattn_decode_params base = db.params(b, 1, kPage);
    pdattn_cascade_plan* cp = nullptr;
    PD_OK(pdattn_cascade_plan_create(&base, b.indptr.data(), b.indices.data(), b.lens.data(),
                                     db.indices, 16, &cp));
    pdattn_cascade_info info{};
    PD_OK(pdattn_cascade_plan_get_info(cp, &info));
    pdattn_workspace ws{};
    PD_OK(pdattn_cascade_decode(cp, db.out, db.lse, &ws, nullptr));
    char tag[160];
    std::snprintf(tag, sizeof tag, "%s cascade (prefix %d tokens, use %d)", name, info.prefix_tokens, info.use);
    check(tag, b, db);
    if (info.use != 1) {
        std::printf("%s: the cascade plan did not use the shared prefix  FAIL\n", name);
        ++g_failures;
    }
    pdattn_cascade_plan_destroy(cp);
    pdattn_workspace_release(&ws);
}

}  // namespace

extern "C" int pdattn_drop_in_checks(void) {
    g_failures = 0;
    int n = 0;
    HIP_OK(hipGetDeviceCount(&n));
    if (n < 1) {
        std::fprintf(stderr, "no GPU\n");
        return -1;
    }
    // the reference's correctness cases (01:750-755), seed 7 (01:758)
    decode_case("MHA lens {1,17,1000}", {1, 17, 1000}, 8, 8, 7);
    decode_case("GQA G=4 lens {5,300,2049,4096}", {5, 300, 2049, 4096}, 32, 8, 7);
    decode_case("GQA G=8 lens {33,777}", {33, 777}, 16, 2, 7);
    decode_case("G=2 page boundaries {16,32,48,4097}", {16, 32, 48, 4097}, 4, 2, 7);
    // shared-prefix cases (01:782-787), seed 13, min_prefix 16
    cascade_case("cascade MHA prefix 64", 64, {1, 17, 40}, 8, 8, 13);
    cascade_case("cascade G=4 prefix 1024 x 40", 1024, std::vector<int>(40, 77), 32, 8, 13);
    cascade_case("cascade G=8 prefix 256", 256, {100, 3}, 16, 2, 13);
    // no shared page: the cascade planner reports 0 shared pages (01:810-815)
    {
        const Batch b = make_batch({1000, 1000, 1000, 1000}, 32, 8, 3);
        const int pp = pdattn_shared_prefix_pages(b.indptr.data(), b.indices.data(), b.B);
        std::printf("%-52s %d shared pages  %s\n", "unshared batch shared_prefix_pages", pp, pp == 0 ? "PASS" : "FAIL");
        if (pp != 0) ++g_failures;
    }
    std::printf("%s: %d failure(s)\n", g_failures ? "FAILED" : "ALL PASS", g_failures);
    std::fflush(stdout);
    return g_failures;
}

#ifdef DROP_IN_MAIN
int main() { return pdattn_drop_in_checks() == 0 ? 0 : 1; }
#endif
