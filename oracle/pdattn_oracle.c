/*
 * pdattn_oracle.c -- fp64 CPU restatement of the paged split-KV GQA decode attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP library is compared against.
 * Nothing in the product library links, loads or calls it; only the tests, the smoke check and
 * the CPU-baseline leg of the benchmark do.
 *
 * Every function restates an algorithm of the reference (qilem/cuda-kernel-lab,
 * 01_decode_attention.cu) from its source; the file:line each one follows is given at the
 * function. Arithmetic is done in double throughout, including the output accumulation (the
 * reference sums `out` in float at 01_decode_attention.cu:396; that deviation is deliberate).
 *
 * Layouts (identical to the reference, 01_decode_attention.cu:5-9, 112):
 *   q        [B, Hq, 128]                 fp16 bits (uint16)
 *   k, v     [num_pages, 16, Hkv, 128]    fp16 bits; element (page, slot, kvh, d) at
 *                                          ((page*16 + slot)*Hkv + kvh)*128 + d
 *   indptr   [B+1], indices [nnz], last [B]  int32 CSR page table
 *   out      [B, Hq, 128] double, lse [B, Hq] double (natural log of the scaled scores)
 *
 * Fault injection (oracle_set_fault) exists so that the tests can show that each pinning
 * check catches a plausible mistake; it is off (0) unless a test turns it on.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HEAD_DIM 128
#define PAGE 16

/* ---- fault injection (test-only) ------------------------------------------------------- */
enum {
    FAULT_NONE = 0,
    FAULT_PAGE_OFF_BY_ONE = 1,  /* reads the next page of the sequence (wrapping)             */
    FAULT_KVH_MODULO = 2,       /* maps q head h to kv head h % Hkv instead of h / G          */
    FAULT_NO_SCALE = 3,         /* drops sm_scale                                             */
    FAULT_FULL_LAST_PAGE = 4,   /* ignores kv_last_page_len (treats the last page as full)    */
    FAULT_LSE_NO_MAX = 5,       /* lse forgets to add back the running max                    */
    FAULT_SLOT_TRANSPOSE = 6,   /* swaps the slot and kv-head strides of the page layout      */
    FAULT_MERGE_NO_WEIGHT = 7,  /* merge averages partial outputs without exp(lse) weights    */
    FAULT_HALF_TRUNC = 8,       /* double->half truncates instead of rounding to nearest even */
    FAULT_PREFIX_NO_PRIVATE = 9 /* shared-prefix detection lets the last page be shared       */
};
static int g_fault = FAULT_NONE;
void oracle_set_fault(int code) { g_fault = code; }
int oracle_get_fault(void) { return g_fault; }

/* ---- binary16 codec ----------------------------------------------------------------------
 * IEEE 754 binary16: 1 sign bit, 5 exponent bits (bias 15), 10 fraction bits. Written from
 * the format definition; pinned in the tests against numpy's float16 on all 65536 patterns. */
double oracle_half_to_double(uint16_t h) {
    int sign = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);                 /* zero / subnormal */
    else if (e == 31) v = m ? NAN : INFINITY;              /* inf / nan        */
    else v = ldexp((double)(1024 + m), e - 25);            /* normal           */
    return sign ? -v : v;
}

uint16_t oracle_double_to_half(double x) {
    uint16_t sign = (uint16_t)(signbit(x) ? 0x8000 : 0);
    double a = fabs(x);
    if (isnan(x)) return 0x7e00;
    if (a == 0.0) return sign;
    int e2;
    frexp(a, &e2);                 /* a = f * 2^e2, f in [0.5, 1) -> floor(log2 a) = e2 - 1 */
    int E = e2 - 1;
    int qexp = (E < -14) ? -24 : E - 10;                   /* quantum of the target binade */
    double scaled = ldexp(a, -qexp);                       /* exact: power-of-two scaling  */
    double n = (g_fault == FAULT_HALF_TRUNC) ? floor(scaled) : nearbyint(scaled); /* RNE */
    if (E < -14) return (uint16_t)(sign | (uint16_t)n);    /* subnormal; n==1024 -> min normal */
    if (n >= 2048.0) { n = 1024.0; E += 1; }
    if (E > 15) return (uint16_t)(sign | 0x7c00);          /* overflow -> inf */
    return (uint16_t)(sign | (uint16_t)((E + 15) << 10) | (uint16_t)((int)n - 1024));
}

/* Table of all 65536 binary16 values as double, filled once from oracle_half_to_double; the
 * decode loops read it instead of decoding each element again. */
static double g_h2d[65536];
static pthread_once_t g_h2d_once = PTHREAD_ONCE_INIT;
static void h2d_init(void) {
    for (int i = 0; i < 65536; i++) g_h2d[i] = oracle_half_to_double((uint16_t)i);
}
static inline double h2d(uint16_t h) { return g_h2d[h]; }

/* ---- page-table helpers ------------------------------------------------------------------ */
/* Sequence length from the CSR page table: (npages-1)*16 + last, 0 when the sequence has no
 * pages. Follows 01_decode_attention.cu:93-95. */
static int seq_len(const int32_t* indptr, const int32_t* last, int b) {
    int np = indptr[b + 1] - indptr[b];
    if (np <= 0) return 0;
    int l = (g_fault == FAULT_FULL_LAST_PAGE) ? PAGE : last[b];
    return (np - 1) * PAGE + l;
}

/* Element offset of row (key) `key` of sequence b, kv head kvh. Follows 01:111-112 / 01:383-384. */
static size_t kv_offset(const int32_t* indptr, const int32_t* indices, int Hkv, int b, int key, int kvh) {
    int pos = indptr[b] + key / PAGE;
    if (g_fault == FAULT_PAGE_OFF_BY_ONE) pos = indptr[b] + (key / PAGE + 1) % (indptr[b + 1] - indptr[b]);
    int page = indices[pos];
    if (g_fault == FAULT_SLOT_TRANSPOSE)
        return (((size_t)page * Hkv + kvh) * PAGE + key % PAGE) * HEAD_DIM;
    return (((size_t)page * PAGE + key % PAGE) * Hkv + kvh) * HEAD_DIM;
}

static int kv_head_of(int h, int Hq, int Hkv) {
    int G = Hq / Hkv;
    return (g_fault == FAULT_KVH_MODULO) ? h % Hkv : h / G;
}

/* Attention of one (sequence, q head) row over keys [kbeg, kend), in double.
 * o = sum_j softmax(s)_j v_j, lse = m + ln(sum_j exp(s_j - m)), s_j = scale * q.k_j.
 * Empty range -> o = 0, lse = -inf (01:228-235). Follows 01:370-400. */
static void attend_row(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       const int32_t* indptr, const int32_t* indices,
                       int Hq, int Hkv, int b, int h, int kbeg, int kend, double scale,
                       double* o, double* lse, double* sbuf) {
    int kvh = kv_head_of(h, Hq, Hkv);
    const uint16_t* qv = q + ((size_t)b * Hq + h) * HEAD_DIM;
    double qd[HEAD_DIM];
    for (int d = 0; d < HEAD_DIM; d++) qd[d] = h2d(qv[d]);
    for (int d = 0; d < HEAD_DIM; d++) o[d] = 0.0;
    if (kend <= kbeg) { *lse = -INFINITY; return; }
    double m = -INFINITY;
    for (int key = kbeg; key < kend; key++) {
        size_t off = kv_offset(indptr, indices, Hkv, b, key, kvh);
        double acc = 0.0;
        for (int d = 0; d < HEAD_DIM; d++) acc += qd[d] * h2d(k[off + d]);
        double s = (g_fault == FAULT_NO_SCALE) ? acc : acc * scale;
        sbuf[key - kbeg] = s;
        if (s > m) m = s;
    }
    double den = 0.0;
    for (int key = kbeg; key < kend; key++) {
        double e = exp(sbuf[key - kbeg] - m);
        sbuf[key - kbeg] = e;
        den += e;
    }
    for (int key = kbeg; key < kend; key++) {
        size_t off = kv_offset(indptr, indices, Hkv, b, key, kvh);
        double w = sbuf[key - kbeg] / den;
        for (int d = 0; d < HEAD_DIM; d++) o[d] += w * h2d(v[off + d]);
    }
    *lse = (g_fault == FAULT_LSE_NO_MAX) ? log(den) : m + log(den);
}

static int max_seq_len(const int32_t* indptr, const int32_t* last, int B) {
    int mx = 0;
    for (int b = 0; b < B; b++) { int L = seq_len(indptr, last, b); if (L > mx) mx = L; }
    return mx;
}

/* Full decode attention for every (b, q head), keys [kv_start, seq_len). Follows
 * 01_decode_attention.cu:370-400 (with the kv_start skip of 01:96). Rows are split over
 * `threads` POSIX threads (1 = the reference's single-threaded loop). */
typedef struct {
    const uint16_t *q, *k, *v;
    const int32_t *indptr, *indices, *last;
    int B, Hq, Hkv, kv_start, row_begin, row_end;
    double scale;
    double *out, *lse;
} decode_job;

static void* decode_worker(void* arg) {
    decode_job* j = (decode_job*)arg;
    int mx = max_seq_len(j->indptr, j->last, j->B);
    double* sbuf = (double*)malloc(sizeof(double) * (size_t)(mx > 0 ? mx : 1));
    for (int row = j->row_begin; row < j->row_end; row++) {
        int b = row / j->Hq, h = row % j->Hq;
        int L = seq_len(j->indptr, j->last, b);
        attend_row(j->q, j->k, j->v, j->indptr, j->indices, j->Hq, j->Hkv, b, h,
                   j->kv_start, L, j->scale, j->out + (size_t)row * HEAD_DIM, j->lse + row, sbuf);
    }
    free(sbuf);
    return NULL;
}

void oracle_decode_mt(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      const int32_t* indptr, const int32_t* indices, const int32_t* last,
                      int B, int Hq, int Hkv, int kv_start, double sm_scale,
                      double* out, double* lse, int threads) {
    pthread_once(&g_h2d_once, h2d_init);
    int rows = B * Hq;
    if (threads < 1) threads = 1;
    if (threads > rows) threads = rows > 0 ? rows : 1;
    decode_job* jobs = (decode_job*)calloc((size_t)threads, sizeof(decode_job));
    pthread_t* tids = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    for (int t = 0; t < threads; t++) {
        decode_job* j = &jobs[t];
        j->q = q; j->k = k; j->v = v; j->indptr = indptr; j->indices = indices; j->last = last;
        j->B = B; j->Hq = Hq; j->Hkv = Hkv; j->kv_start = kv_start; j->scale = sm_scale;
        j->out = out; j->lse = lse;
        j->row_begin = (int)((long long)rows * t / threads);
        j->row_end = (int)((long long)rows * (t + 1) / threads);
        if (threads == 1) decode_worker(j);
        else pthread_create(&tids[t], NULL, decode_worker, j);
    }
    if (threads > 1)
        for (int t = 0; t < threads; t++) pthread_join(tids[t], NULL);
    free(jobs);
    free(tids);
}

void oracle_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                   const int32_t* indptr, const int32_t* indices, const int32_t* last,
                   int B, int Hq, int Hkv, int kv_start, double sm_scale,
                   double* out, double* lse) {
    oracle_decode_mt(q, k, v, indptr, indices, last, B, Hq, Hkv, kv_start, sm_scale, out, lse, 1);
}

/* Per-chunk partial states with the reference's uniform chunking: chunk c of every sequence
 * covers keys [kv_start + c*chunk_tokens, min(seq_len, kv_start + (c+1)*chunk_tokens)), and its
 * partial is the normalized (o, lse) of that range; an empty range gives (0, -inf).
 * Partial row layout: part_o[(row*part_stride + chunk_base + c)*128 + d],
 * part_lse[row*part_stride + chunk_base + c], row = b*Hq + h.
 * Follows 01_decode_attention.cu:88-97 and 228-235. */
void oracle_partials(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                     const int32_t* indptr, const int32_t* indices, const int32_t* last,
                     int B, int Hq, int Hkv, int num_chunks, int chunk_tokens, int kv_start,
                     int chunk_base, int part_stride, double sm_scale,
                     double* part_o, double* part_lse) {
    pthread_once(&g_h2d_once, h2d_init);
    double* sbuf = (double*)malloc(sizeof(double) * (size_t)(chunk_tokens > 0 ? chunk_tokens : 1));
    for (int b = 0; b < B; b++) {
        int L = seq_len(indptr, last, b);
        for (int h = 0; h < Hq; h++) {
            size_t row = (size_t)b * Hq + h;
            for (int c = 0; c < num_chunks; c++) {
                int kbeg = kv_start + c * chunk_tokens;
                int kend = kbeg + chunk_tokens < L ? kbeg + chunk_tokens : L;
                size_t slot = row * part_stride + chunk_base + c;
                attend_row(q, k, v, indptr, indices, Hq, Hkv, b, h, kbeg, kend, sm_scale,
                           part_o + slot * HEAD_DIM, part_lse + slot, sbuf);
            }
        }
    }
    free(sbuf);
}

/* Log-sum-exp merge of `num_chunks` partial states per row, in fixed chunk order.
 * m = max_c lse_c; if m = -inf: o = 0, lse = -inf; else w_c = exp(lse_c - m),
 * o = sum_c w_c o_c / sum_c w_c, lse = m + ln(sum_c w_c). Follows 01_decode_attention.cu:238-255. */
void oracle_merge(const double* part_o, const double* part_lse, int rows, int num_chunks,
                  double* out, double* lse) {
    for (int r = 0; r < rows; r++) {
        const double* pl = part_lse + (size_t)r * num_chunks;
        double m = -INFINITY;
        for (int c = 0; c < num_chunks; c++) if (pl[c] > m) m = pl[c];
        double wsum = 0.0, acc[HEAD_DIM];
        for (int d = 0; d < HEAD_DIM; d++) acc[d] = 0.0;
        if (m != -INFINITY) {
            for (int c = 0; c < num_chunks; c++) {
                double w = (g_fault == FAULT_MERGE_NO_WEIGHT) ? 1.0 : exp(pl[c] - m);
                if (pl[c] == -INFINITY) w = 0.0;
                wsum += w;
                const double* po = part_o + ((size_t)r * num_chunks + c) * HEAD_DIM;
                for (int d = 0; d < HEAD_DIM; d++) acc[d] += w * po[d];
            }
        }
        for (int d = 0; d < HEAD_DIM; d++) out[(size_t)r * HEAD_DIM + d] = wsum > 0.0 ? acc[d] / wsum : 0.0;
        lse[r] = wsum > 0.0 ? m + log(wsum) : -INFINITY;
    }
}

/* Longest run of physical pages that every sequence starts with, keeping at least one private
 * page per sequence; 0 when B < 2. Follows 01_decode_attention.cu:634-646. */
int oracle_shared_prefix_pages(const int32_t* indptr, const int32_t* indices, int B) {
    if (B < 2) return 0;
    int keep = (g_fault == FAULT_PREFIX_NO_PRIVATE) ? 0 : 1;
    for (int P = 0;; P++) {
        for (int b = 0; b < B; b++)
            if (P >= indptr[b + 1] - indptr[b] - keep) return P;
        int pg = indices[indptr[0] + P];
        for (int b = 1; b < B; b++)
            if (indices[indptr[b] + P] != pg) return P;
    }
}

/* The reference's uniform split rule, given the number of resident blocks of one wave
 * (SMs x occupancy): chunks = force, or min(max(1, resident/(B*Hkv)), max(1, ceil(max_len/256)));
 * chunk_tokens = ceil(ceil(max_len/chunks)/32)*32; num_chunks = ceil(max_len/chunk_tokens).
 * Follows 01_decode_attention.cu:289-312. Used only to compare chunk counts with the reference. */
void oracle_plan_chunks_ref(int resident_blocks, int B, int Hkv, int max_len, int force_chunks,
                            int* num_chunks, int* chunk_tokens) {
    int chunks;
    if (force_chunks > 0) {
        chunks = force_chunks;
    } else {
        int want = resident_blocks / (B * Hkv);
        if (want < 1) want = 1;
        int cap = (max_len + 255) / 256;
        if (cap < 1) cap = 1;
        chunks = want < cap ? want : cap;
    }
    int per = (max_len + chunks - 1) / chunks;
    int tokens = ((per + 31) / 32) * 32;
    if (tokens < 32) tokens = 32;
    *chunk_tokens = tokens;
    *num_chunks = (max_len + tokens - 1) / tokens;
}
