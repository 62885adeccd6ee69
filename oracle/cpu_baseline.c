/* cpu_baseline.c - the reference's CPU expert path as a timed baseline.
 * TEST INFRASTRUCTURE ONLY: bench.py times it beside the GPU path; tests check it against the
 * scalar oracle. It restates:
 *   - the persistent worker pool: workers park on a condition variable, a generation counter
 *     publishes each job, rows are claimed 16 at a time with an atomic counter
 *     (runtime/src/expert_pool.rs:86-136, 357-393, 408-447);
 *   - caller-thread Q8_0 quantisation, once per activation row (expert_pool.rs:311-320);
 *   - the AVX2+FMA Q4xQ8 dot the reference selects on AVX2 hosts (expert_kernel.rs:85-95,
 *     163-191), or the scalar dot (147-161) when the host lacks AVX2/FMA;
 *   - router, selection, plan, GeGLU and combine on the caller thread (runtime/src/exec.rs:456-475,
 *     572-640). */
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "moe_oracle.h"

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define QK 32
#define Q4_BLOCK 18
#define Q8_BLOCK 34
#define CHUNK 16

typedef struct {
    const uint8_t *w; /* n_out Q4_0 rows */
    const uint8_t *xq; /* n_in Q8_0 rows */
    size_t n_out, n_in, y_off;
} seg_t;

typedef struct {
    const seg_t *segs;
    const size_t *starts; /* nseg + 1 */
    size_t nseg, k, total;
    float *y;
    atomic_size_t next;
} job_t;

struct cpb_pool {
    int n;
    pthread_t *threads;
    pthread_mutex_t mu;
    pthread_cond_t wake, done;
    uint64_t generation;
    int remaining, stop;
    job_t *job;
    /* caller scratch, grown on demand and reused */
    size_t cap_pairs, cap_d, cap_ff, cap_exp;
    float *logits, *gu, *h, *y, *xin;
    uint8_t *xq, *hq;
    uint32_t *order, *pos_of, *gs;
    seg_t *segs;
    size_t *starts;
    /* wall time of the expert part of every cpb_moe_layer call so far (plan, quantisation, the two
       pooled GEMV segments, GeGLU, combine: what the reference's CPU expert span covers, without the
       router and selection that run before it on the caller thread) */
    uint64_t expert_ns;
};

static uint64_t now_ns(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

uint64_t cpb_expert_ns(const cpb_pool *p) { return p ? p->expert_ns : 0; }

static int g_avx2 = -1;

int cpb_uses_avx2(void) {
    if (g_avx2 < 0) {
#if defined(__x86_64__)
        __builtin_cpu_init();
        g_avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
#else
        g_avx2 = 0;
#endif
    }
    return g_avx2;
}

#if defined(__x86_64__)
/* runtime/src/expert_kernel.rs:163-191 */
__attribute__((target("avx2,fma"))) static float dot_avx2_q8(const uint8_t *row, const uint8_t *xq, size_t k) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i low = _mm256_set1_epi8(15);
    const __m256i bias = _mm256_set1_epi8(8);
    const __m256i ones = _mm256_set1_epi16(1);
    for (size_t b = 0; b < k / QK; ++b) {
        const uint8_t *w = row + b * Q4_BLOCK;
        const uint8_t *x = xq + b * Q8_BLOCK;
        float d = orc_f16_to_f32((uint16_t)(w[0] | (w[1] << 8))) * orc_f16_to_f32((uint16_t)(x[0] | (x[1] << 8)));
        __m128i packed = _mm_loadu_si128((const __m128i *)(w + 2));
        __m256i both = _mm256_set_m128i(_mm_srli_epi16(packed, 4), packed);
        __m256i qw = _mm256_sub_epi8(_mm256_and_si256(both, low), bias);
        __m256i qx = _mm256_loadu_si256((const __m256i *)(x + 2));
        __m256i products = _mm256_maddubs_epi16(_mm256_sign_epi8(qw, qw), _mm256_sign_epi8(qx, qw));
        __m256i sumi = _mm256_madd_epi16(products, ones);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    float sums[8];
    _mm256_storeu_ps(sums, acc);
    float s = -0.0f;
    for (int i = 0; i < 8; ++i) s += sums[i];
    return s;
}
#endif

static float dot_q8(const uint8_t *row, const uint8_t *xq, size_t k) {
#if defined(__x86_64__)
    if (g_avx2 > 0) return dot_avx2_q8(row, xq, k);
#endif
    return orc_dot_q8_scalar(row, xq, k);
}

/* runtime/src/expert_pool.rs:86-136 */
static void job_execute(job_t *job) {
    size_t row_bytes = job->k / QK * Q4_BLOCK;
    size_t q_bytes = job->k / QK * Q8_BLOCK;
    for (;;) {
        size_t a = atomic_fetch_add_explicit(&job->next, CHUNK, memory_order_relaxed);
        if (a >= job->total) break;
        size_t b = a + CHUNK < job->total ? a + CHUNK : job->total;
        size_t si = 0;
        while (job->starts[si + 1] <= a) ++si;
        for (size_t g = a; g < b; ++g) {
            while (g >= job->starts[si + 1]) ++si;
            const seg_t *s = &job->segs[si];
            size_t r = g - job->starts[si];
            const uint8_t *w = s->w + r * row_bytes;
            for (size_t t = 0; t < s->n_in; ++t) job->y[s->y_off + t * s->n_out + r] = dot_q8(w, s->xq + t * q_bytes, job->k);
        }
    }
}

/* runtime/src/expert_pool.rs:408-447 (sleep policy: park on the condition variable) */
static void *worker_main(void *arg) {
    cpb_pool *p = (cpb_pool *)arg;
    uint64_t seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        while (!p->stop && p->generation == seen) pthread_cond_wait(&p->wake, &p->mu);
        if (p->stop) {
            pthread_mutex_unlock(&p->mu);
            return NULL;
        }
        seen = p->generation;
        job_t *job = p->job;
        pthread_mutex_unlock(&p->mu);
        job_execute(job);
        pthread_mutex_lock(&p->mu);
        if (--p->remaining == 0) pthread_cond_signal(&p->done);
        pthread_mutex_unlock(&p->mu);
    }
}

/* runtime/src/expert_pool.rs:357-393 */
static void pool_submit(cpb_pool *p, job_t *job) {
    pthread_mutex_lock(&p->mu);
    p->remaining = p->n;
    p->job = job;
    p->generation++;
    pthread_cond_broadcast(&p->wake);
    while (p->remaining > 0) pthread_cond_wait(&p->done, &p->mu);
    p->job = NULL;
    pthread_mutex_unlock(&p->mu);
}

cpb_pool *cpb_create(int threads) {
    if (threads < 1 || threads > 256) return NULL;
    cpb_uses_avx2();
    cpb_pool *p = (cpb_pool *)calloc(1, sizeof(cpb_pool));
    p->n = threads;
    p->threads = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->wake, NULL);
    pthread_cond_init(&p->done, NULL);
    for (int i = 0; i < threads; ++i) pthread_create(&p->threads[i], NULL, worker_main, p);
    return p;
}

void cpb_destroy(cpb_pool *p) {
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    p->stop = 1;
    pthread_cond_broadcast(&p->wake);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->n; ++i) pthread_join(p->threads[i], NULL);
    pthread_mutex_destroy(&p->mu);
    pthread_cond_destroy(&p->wake);
    pthread_cond_destroy(&p->done);
    free(p->threads);
    free(p->logits);
    free(p->gu);
    free(p->h);
    free(p->y);
    free(p->xin);
    free(p->xq);
    free(p->hq);
    free(p->order);
    free(p->pos_of);
    free(p->gs);
    free(p->segs);
    free(p->starts);
    free(p);
}

int cpb_threads(const cpb_pool *p) { return p ? p->n : 0; }

static void reserve(cpb_pool *p, size_t pairs, size_t n_tok, size_t n_exp, size_t d, size_t ff) {
    if (pairs <= p->cap_pairs && d <= p->cap_d && ff <= p->cap_ff && n_exp <= p->cap_exp && n_tok <= p->cap_pairs)
        return;
    size_t np = pairs > p->cap_pairs ? pairs : p->cap_pairs;
    size_t nd = d > p->cap_d ? d : p->cap_d;
    size_t nf = ff > p->cap_ff ? ff : p->cap_ff;
    size_t ne = n_exp > p->cap_exp ? n_exp : p->cap_exp;
    p->logits = (float *)realloc(p->logits, np * ne * sizeof(float));
    p->xin = (float *)realloc(p->xin, np * nd * sizeof(float));
    p->gu = (float *)realloc(p->gu, np * 2 * nf * sizeof(float));
    p->h = (float *)realloc(p->h, np * nf * sizeof(float));
    p->y = (float *)realloc(p->y, np * nd * sizeof(float));
    p->xq = (uint8_t *)realloc(p->xq, np * (nd / QK) * Q8_BLOCK);
    p->hq = (uint8_t *)realloc(p->hq, np * (nf / QK) * Q8_BLOCK);
    p->order = (uint32_t *)realloc(p->order, np * sizeof(uint32_t));
    p->pos_of = (uint32_t *)realloc(p->pos_of, np * sizeof(uint32_t));
    p->gs = (uint32_t *)realloc(p->gs, (ne + 1) * sizeof(uint32_t));
    p->segs = (seg_t *)realloc(p->segs, ne * sizeof(seg_t));
    p->starts = (size_t *)realloc(p->starts, (ne + 1) * sizeof(size_t));
    p->cap_pairs = np;
    p->cap_d = nd;
    p->cap_ff = nf;
    p->cap_exp = ne;
}

/* runtime/src/expert_pool.rs:282-355 over the groups of the plan. */
static void run_segments(cpb_pool *p, const uint8_t *const *w, size_t row_bytes_of_k, size_t n_out, size_t k,
                         const uint8_t *xq, size_t q_row_bytes, const uint32_t *gs, size_t n_exp, float *y) {
    size_t nseg = 0, total = 0;
    for (size_t e = 0; e < n_exp; ++e) {
        size_t st = gs[e], len = gs[e + 1] - gs[e];
        if (len == 0) continue;
        seg_t *s = &p->segs[nseg];
        s->w = w[e];
        s->xq = xq + st * q_row_bytes;
        s->n_out = n_out;
        s->n_in = len;
        s->y_off = st * n_out;
        p->starts[nseg] = total;
        total += n_out;
        ++nseg;
    }
    p->starts[nseg] = total;
    (void)row_bytes_of_k;
    job_t job;
    job.segs = p->segs;
    job.starts = p->starts;
    job.nseg = nseg;
    job.k = k;
    job.total = total;
    job.y = y;
    atomic_init(&job.next, 0);
    if (total) pool_submit(p, &job);
}

int cpb_moe_layer(cpb_pool *p, const float *w_r, const float *bias, const uint8_t *const *gate_up,
                  const uint8_t *const *down, const float *down_scale, const float *x, size_t n_tok,
                  size_t n_exp, size_t d, size_t ff, size_t used, uint32_t *ids, float *weights, float *out) {
    size_t pairs = n_tok * used;
    reserve(p, pairs, n_tok, n_exp, d, ff);
    /* router and selection on the caller thread (exec.rs:493-517) */
    orc_router_logits(w_r, bias, x, n_tok, n_exp, d, p->logits);
    orc_select_experts(p->logits, n_tok, n_exp, used, ids, weights);
    for (size_t i = 0; i < pairs; ++i)
        if (ids[i] >= n_exp || !gate_up[ids[i]] || !down[ids[i]]) return -1;
    const uint64_t t0 = now_ns();
    orc_moe_plan(ids, pairs, n_exp, p->order, p->pos_of, p->gs);
    size_t xq_bytes = d / QK * Q8_BLOCK, hq_bytes = ff / QK * Q8_BLOCK;
    /* gather + caller-thread quantisation of each segment row */
    for (size_t k = 0; k < pairs; ++k) orc_quantize_q8_0(x + (p->order[k] / used) * d, p->xq + k * xq_bytes, d);
    run_segments(p, gate_up, d / QK * Q4_BLOCK, 2 * ff, d, p->xq, xq_bytes, p->gs, n_exp, p->gu);
    /* GeGLU on the caller (exec.rs:606-611) and quantisation of the down inputs */
    for (size_t k = 0; k < pairs; ++k) {
        for (size_t j = 0; j < ff; ++j) p->h[k * ff + j] = orc_gelu(p->gu[k * 2 * ff + j]) * p->gu[k * 2 * ff + ff + j];
        orc_quantize_q8_0(p->h + k * ff, p->hq + k * hq_bytes, ff);
    }
    run_segments(p, down, ff / QK * Q4_BLOCK, d, ff, p->hq, hq_bytes, p->gs, n_exp, p->y);
    /* slot-order combine (exec.rs:626-638) */
    for (size_t t = 0; t < n_tok; ++t) {
        float *o = out + t * d;
        for (size_t j = 0; j < used; ++j) {
            uint32_t ex = ids[t * used + j];
            float wt = weights[t * used + j];
            float ds = down_scale ? down_scale[ex] : 1.0f;
            const float *yy = p->y + (size_t)p->pos_of[t * used + j] * d;
            if (j == 0)
                for (size_t i = 0; i < d; ++i) o[i] = yy[i] * ds * wt;
            else
                for (size_t i = 0; i < d; ++i) o[i] += yy[i] * ds * wt;
        }
    }
    p->expert_ns += now_ns() - t0;
    return 0;
}
