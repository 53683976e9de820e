/*
 * rh_avx2.c -- CPU baseline only: a C restatement, with AVX2 intrinsics, of
 * the Q4_K and Q6_K kernels rusticide runs on x86 (the avx2 adapter,
 * crates/rusticide-kernels/src/adapter.rs:86-169, which repacks a matrix into
 * eight-row units when it is prepared, adapter.rs:70-83).
 *
 * Test infrastructure: only the tests and bench.py's cpu_baseline leg call
 * it. It times the reference's fastest CPU path on the GPU box's host cores
 * and is checked bit for bit against the portable restatement in
 * rh_oracle.c (tests/test_avx2_baseline.py); the product never runs it.
 *
 * Layouts (crates/rusticide-simd/src/group/q4_k.rs:5-34,
 * group/q6_k.rs:5-35): unit k of a group of eight rows holds block k of each
 * row, interleaved so that 32 bytes hold the same four bytes of all eight
 * rows.
 *   Q4_K (1152 bytes): d of row r at 2r, dmin at 16 + 2r, packed scale byte
 *     i at 32 + 8i + r, quant bytes 4c..4c+3 at 128 + 32c + 4r.
 *   Q6_K (1680 bytes): low-bit bytes 4c.. at 32c + 4r, high-bit bytes 4c..
 *     at 1024 + 32c + 4r, scale s at 1536 + 8s + r, d at 1664 + 2r.
 * Kernels (crates/rusticide-simd/src/avx2/q4_k/vector.rs:56-178,
 * avx2/q6_k/vector.rs:84-209): one i32 lane per row; vpmaddubsw of the
 * unsigned weights (Q6_K: their magnitudes, the activation carrying the
 * sign) against four broadcast activation bytes, vpmaddwd by the run scale,
 * the per-block float combine in the portable kernels' order and roundings
 * (int_dot.rs:169 and :203). The reference's views refuse an input holding
 * the quant -128, which the sign trick cannot negate (group_views.rs:6);
 * Q8_K clamps its quants to [-127, 127] (portable/q8.rs:113-115), so the
 * same guard here never fires for these kernels and stays as a guard.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "rh_oracle.h"

#define AVX2 __attribute__((target("avx2,fma")))

enum { ROWS = 8, UNIT_Q4 = 1152, UNIT_Q6 = 1680 };

struct orc_avx2_matrix {
    uint32_t type_id;
    size_t rows, nblocks, unit;
    uint8_t *units; /* [rows / 8][nblocks][unit] */
};

int orc_avx2_available(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

orc_avx2_matrix *orc_avx2_prepare(uint32_t type_id, const uint8_t *data, size_t rows, size_t row_bytes)
{
    const size_t bb = type_id == 12 ? 144 : type_id == 14 ? 210 : 0;
    if (!bb || rows == 0 || rows % ROWS || row_bytes % bb || !orc_avx2_available()) return NULL;
    orc_avx2_matrix *m = (orc_avx2_matrix *)calloc(1, sizeof(*m));
    if (!m) return NULL;
    m->type_id = type_id;
    m->rows = rows;
    m->nblocks = row_bytes / bb;
    m->unit = type_id == 12 ? UNIT_Q4 : UNIT_Q6;
    m->units = (uint8_t *)aligned_alloc(64, (rows / ROWS) * m->nblocks * m->unit);
    if (!m->units) {
        free(m);
        return NULL;
    }
    for (size_t g = 0; g < rows / ROWS; g++)
        for (size_t k = 0; k < m->nblocks; k++) {
            uint8_t *u = m->units + (g * m->nblocks + k) * m->unit;
            for (size_t r = 0; r < ROWS; r++) {
                const uint8_t *b = data + (g * ROWS + r) * row_bytes + k * bb;
                if (type_id == 12) {
                    memcpy(u + 2 * r, b, 2);
                    memcpy(u + 16 + 2 * r, b + 2, 2);
                    for (size_t i = 0; i < 12; i++) u[32 + 8 * i + r] = b[4 + i];
                    for (size_t c = 0; c < 32; c++) memcpy(u + 128 + 32 * c + 4 * r, b + 16 + 4 * c, 4);
                } else {
                    for (size_t c = 0; c < 32; c++) memcpy(u + 32 * c + 4 * r, b + 4 * c, 4);
                    for (size_t c = 0; c < 16; c++) memcpy(u + 1024 + 32 * c + 4 * r, b + 128 + 4 * c, 4);
                    for (size_t s = 0; s < 16; s++) u[1536 + 8 * s + r] = b[192 + s];
                    memcpy(u + 1664 + 2 * r, b + 208, 2);
                }
            }
        }
    return m;
}

void orc_avx2_free(orc_avx2_matrix *m)
{
    if (!m) return;
    free(m->units);
    free(m);
}

/* Eight f16 values (one per row) widened as the reference's scalar
 * f16_to_f32 (avx2/vector.rs:15-35): magnitude shifted into place and
 * rebiased by a multiply, infinities and NaN passed through. */
static AVX2 __m256 halves8(const uint8_t *p)
{
    const __m256i bits = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)p));
    const __m256i mag = _mm256_and_si256(bits, _mm256_set1_epi32(0x7fff));
    const __m256i shifted = _mm256_slli_epi32(mag, 13);
    const __m256 rebiased = _mm256_mul_ps(_mm256_castsi256_ps(shifted), _mm256_castsi256_ps(_mm256_set1_epi32(0x77800000)));
    const __m256i special = _mm256_cmpgt_epi32(mag, _mm256_set1_epi32(0x7bff));
    const __m256i widened = _mm256_blendv_epi8(_mm256_castps_si256(rebiased),
                                               _mm256_or_si256(shifted, _mm256_set1_epi32(0x7f800000)), special);
    const __m256i sign = _mm256_slli_epi32(_mm256_and_si256(bits, _mm256_set1_epi32(0x8000)), 16);
    return _mm256_castsi256_ps(_mm256_or_si256(widened, sign));
}

static AVX2 __m256i rows_u8(const uint8_t *p)
{
    int64_t v;
    memcpy(&v, p, 8);
    return _mm256_cvtepu8_epi32(_mm_cvtsi64_si128(v));
}

/* Eight signed scale bytes, each in both i16 halves of its row's lane. */
static AVX2 __m256i scale_pairs(const uint8_t *p)
{
    int64_t v;
    memcpy(&v, p, 8);
    const __m256i wide = _mm256_cvtepi8_epi32(_mm_cvtsi64_si128(v));
    return _mm256_blend_epi16(wide, _mm256_slli_epi32(wide, 16), 0xAA);
}

/* One input: quants [nb][256], one scale and eight 32-sums per block. */
typedef struct {
    const int8_t *quants;
    const float *scales; /* per 32-block; the super-block's is entry 8k */
    const int32_t *sums; /* per 32-block */
    size_t nb;
} input_t;

static AVX2 void q4k_group(const uint8_t *units, size_t nblocks, const input_t *in, float *out)
{
    __m256 acc = _mm256_set1_ps(-0.0f);
    const size_t nb = nblocks < in->nb ? nblocks : in->nb;
    const __m256i six = _mm256_set1_epi32(63), four = _mm256_set1_epi32(0x0f), nib = _mm256_set1_epi8(0x0f);
    for (size_t k = 0; k < nb; k++) {
        const uint8_t *u = units + k * UNIT_Q4;
        const __m256 d = halves8(u), dmin = halves8(u + 16);
        __m256i sc[8], mn[8];
        for (int lo = 0; lo < 4; lo++) {
            const __m256i s = rows_u8(u + 32 + 8 * lo), m = rows_u8(u + 32 + 8 * (lo + 4));
            const __m256i hi = rows_u8(u + 32 + 8 * (lo + 8));
            sc[lo] = _mm256_and_si256(s, six);
            mn[lo] = _mm256_and_si256(m, six);
            sc[lo + 4] = _mm256_or_si256(_mm256_and_si256(hi, four), _mm256_slli_epi32(_mm256_srli_epi32(s, 6), 4));
            mn[lo + 4] = _mm256_or_si256(_mm256_srli_epi32(hi, 4), _mm256_slli_epi32(_mm256_srli_epi32(m, 6), 4));
        }
        for (int j = 0; j < 8; j++) sc[j] = _mm256_or_si256(sc[j], _mm256_slli_epi32(sc[j], 16));
        const int8_t *q = in->quants + 256 * k;
        __m256i sum = _mm256_setzero_si256();
        for (int pair = 0; pair < 4; pair++) {
            const uint8_t *raw = u + 128 + 256 * pair;
            for (int half = 0; half < 2; half++) {
                const int run = 2 * pair + half;
                __m256i dots = _mm256_setzero_si256();
                for (int i = 0; i < 8; i++) {
                    __m256i w = _mm256_loadu_si256((const __m256i *)(raw + 32 * i));
                    w = _mm256_and_si256(half ? _mm256_srli_epi16(w, 4) : w, nib);
                    int32_t quad;
                    memcpy(&quad, q + 32 * run + 4 * i, 4);
                    dots = _mm256_add_epi16(dots, _mm256_maddubs_epi16(w, _mm256_set1_epi32(quad)));
                }
                sum = _mm256_add_epi32(sum, _mm256_madd_epi16(dots, sc[run]));
            }
        }
        /* int_dot.rs:169: d8 * d.mul_add(isum, -(dmin * msum)) */
        __m256i msum = _mm256_setzero_si256();
        for (int j = 0; j < 8; j++)
            msum = _mm256_add_epi32(msum, _mm256_mullo_epi32(mn[j], _mm256_set1_epi32(in->sums[8 * k + j])));
        const __m256 neg = _mm256_xor_ps(_mm256_mul_ps(dmin, _mm256_cvtepi32_ps(msum)), _mm256_set1_ps(-0.0f));
        const __m256 term = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(sum), neg);
        acc = _mm256_add_ps(acc, _mm256_mul_ps(term, _mm256_set1_ps(in->scales[8 * k])));
    }
    _mm256_storeu_ps(out, acc);
}

static AVX2 void q6k_group(const uint8_t *units, size_t nblocks, const input_t *in, float *out)
{
    __m256 acc = _mm256_set1_ps(-0.0f);
    const size_t nb = nblocks < in->nb ? nblocks : in->nb;
    const __m256i nib = _mm256_set1_epi8(0x0f), top_mask = _mm256_set1_epi8(0x30), off = _mm256_set1_epi8(32);
    for (size_t k = 0; k < nb; k++) {
        const uint8_t *u = units + k * UNIT_Q6;
        const int8_t *q = in->quants + 256 * k;
        __m256i sum = _mm256_setzero_si256();
        for (int half = 0; half < 2; half++)
            for (int r = 0; r < 4; r++) {
                /* elements 128 half + 32 r + l: ql[64 half + 32 (r & 1) + l]
                 * (high nibble for r >= 2), qh[32 half + l] bits 2r.. */
                const uint8_t *low = u + 256 * (2 * half + (r & 1));
                const uint8_t *high = u + 1024 + 256 * half;
                const int run = 4 * half + r;
                __m256i mag[8], sgn[8];
                for (int i = 0; i < 8; i++) {
                    const __m256i l = _mm256_loadu_si256((const __m256i *)(low + 32 * i));
                    const __m256i h = _mm256_loadu_si256((const __m256i *)(high + 32 * i));
                    const __m256i n = _mm256_and_si256(r < 2 ? l : _mm256_srli_epi16(l, 4), nib);
                    const __m256i t = r == 0 ? _mm256_slli_epi16(h, 4)
                                      : r == 1 ? _mm256_slli_epi16(h, 2)
                                      : r == 2 ? h
                                               : _mm256_srli_epi16(h, 2);
                    sgn[i] = _mm256_sub_epi8(_mm256_or_si256(n, _mm256_and_si256(t, top_mask)), off);
                    mag[i] = _mm256_abs_epi8(sgn[i]);
                }
                for (int h16 = 0; h16 < 2; h16++) {
                    __m256i dots = _mm256_setzero_si256();
                    for (int i = 4 * h16; i < 4 * h16 + 4; i++) {
                        int32_t quad;
                        memcpy(&quad, q + 32 * run + 4 * i, 4);
                        const __m256i a = _mm256_sign_epi8(_mm256_set1_epi32(quad), sgn[i]);
                        dots = _mm256_add_epi16(dots, _mm256_maddubs_epi16(mag[i], a));
                    }
                    sum = _mm256_add_epi32(sum, _mm256_madd_epi16(dots, scale_pairs(u + 1536 + 8 * (2 * run + h16))));
                }
            }
        /* int_dot.rs:203: (d * d8) * isum, then the add, none fused */
        const __m256 dd = _mm256_mul_ps(halves8(u + 1664), _mm256_set1_ps(in->scales[8 * k]));
        acc = _mm256_add_ps(acc, _mm256_mul_ps(dd, _mm256_cvtepi32_ps(sum)));
    }
    _mm256_storeu_ps(out, acc);
}

typedef struct {
    const orc_avx2_matrix *m;
    const input_t *in;
    float *out;
    size_t out_len, groups, per;
    atomic_size_t next;
} work_t;

static void *avx2_worker(void *arg)
{
    work_t *w = (work_t *)arg;
    const size_t tasks = (w->groups + w->per - 1) / w->per;
    for (;;) {
        const size_t t = atomic_fetch_add(&w->next, 1);
        if (t >= tasks) break;
        for (size_t g = t * w->per; g < w->groups && g < (t + 1) * w->per; g++) {
            float rows[ROWS];
            const uint8_t *units = w->m->units + g * w->m->nblocks * w->m->unit;
            if (w->m->type_id == 12) q4k_group(units, w->m->nblocks, w->in, rows);
            else q6k_group(units, w->m->nblocks, w->in, rows);
            for (size_t r = 0; r < ROWS && g * ROWS + r < w->out_len; r++) w->out[g * ROWS + r] = rows[r];
        }
    }
    return NULL;
}

/* A persistent pool of helper threads, as the reference's rayon pool is
 * (matmul.rs:234-247): a call wakes threads - 1 helpers and works beside
 * them, so no call pays for creating threads. Calls are serialized. */
enum { POOL_MAX = 255 };
static struct {
    pthread_mutex_t call, mu;
    pthread_cond_t go, done;
    pthread_t ids[POOL_MAX];
    unsigned long born[POOL_MAX]; /* the generation current when thread i was made */
    int size, active, busy;
    unsigned long gen;
    work_t *w;
} pool = {.call = PTHREAD_MUTEX_INITIALIZER, .mu = PTHREAD_MUTEX_INITIALIZER,
          .go = PTHREAD_COND_INITIALIZER, .done = PTHREAD_COND_INITIALIZER};

static void *pool_main(void *arg)
{
    const int index = (int)(intptr_t)arg;
    pthread_mutex_lock(&pool.mu);
    /* not pool.gen: the call that made this thread may already have
     * advanced it, and that call waits for this thread too */
    unsigned long seen = pool.born[index];
    for (;;) {
        while (pool.gen == seen) pthread_cond_wait(&pool.go, &pool.mu);
        seen = pool.gen;
        work_t *w = index < pool.active ? pool.w : NULL;
        pthread_mutex_unlock(&pool.mu);
        if (w) avx2_worker(w);
        pthread_mutex_lock(&pool.mu);
        if (--pool.busy == 0) pthread_cond_signal(&pool.done);
    }
    return NULL;
}

/* Runs w on the caller and up to helpers pool threads. */
static void pool_run(work_t *w, int helpers)
{
    pthread_mutex_lock(&pool.call);
    pthread_mutex_lock(&pool.mu);
    if (helpers > POOL_MAX) helpers = POOL_MAX;
    while (pool.size < helpers) {
        pool.born[pool.size] = pool.gen;
        if (pthread_create(&pool.ids[pool.size], NULL, pool_main, (void *)(intptr_t)pool.size) != 0) break;
        pool.size++;
    }
    pool.active = helpers < pool.size ? helpers : pool.size;
    pool.busy = pool.size;
    pool.w = w;
    pool.gen++;
    pthread_cond_broadcast(&pool.go);
    pthread_mutex_unlock(&pool.mu);
    avx2_worker(w);
    pthread_mutex_lock(&pool.mu);
    while (pool.busy > 0) pthread_cond_wait(&pool.done, &pool.mu);
    pthread_mutex_unlock(&pool.mu);
    pthread_mutex_unlock(&pool.call);
}

int orc_avx2_matvec(const orc_avx2_matrix *m, const float *x, size_t len, float *out, size_t out_len, int threads)
{
    if (!m || !x || !out || len != m->nblocks * 256) return 0;
    const size_t cap = len / 32 + 1;
    int8_t *quants = (int8_t *)malloc(cap * 32);
    float *scales = (float *)malloc(cap * sizeof(float));
    int32_t *sums = (int32_t *)malloc(cap * sizeof(int32_t));
    int ok = quants && scales && sums;
    size_t n32 = ok ? orc_quantize(ORC_Q8_SUPER_BLOCK, x, len, quants, scales, sums) : 0;
    for (size_t i = 0; ok && i < n32 * 32; i++) ok = quants[i] != -128;
    if (ok) {
        const input_t in = {quants, scales, sums, n32 / 8};
        if (threads <= 0) threads = 1;
        work_t w;
        w.m = m;
        w.in = &in;
        w.out = out;
        w.out_len = out_len;
        w.groups = m->rows / ROWS;
        /* matmul.rs:235-247: 16 tasks a thread, in whole groups */
        const size_t tasks = (size_t)threads * 16;
        w.per = (w.groups + tasks - 1) / tasks;
        if (w.per == 0) w.per = 1;
        atomic_init(&w.next, 0);
        if (threads == 1) avx2_worker(&w);
        else pool_run(&w, threads - 1);
    }
    free(quants);
    free(scales);
    free(sums);
    return ok;
}
