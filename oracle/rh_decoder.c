/*
 * rh_decoder.c -- CPU restatement of rusticide's decoder forward pass and
 * greedy generation, the callers of the quantized matrix product.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the device decoder is compared
 * against. Written from the reference's source, read as text (paths relative
 * to the rusticide repository root):
 *   crates/rusticide-transformer/src/{decoder.rs,attention.rs,feed_forward.rs,
 *     norm.rs,rope.rs,layout.rs}
 *   crates/rusticide-kernels/src/portable/{norm.rs,rope.rs,elementwise.rs}
 *   crates/rusticide-simd/src/float.rs (dot, dot_rows, mix_rows)
 *   crates/rusticide-model/src/{cache.rs,generate.rs}
 *   crates/rusticide-sampling/src/{sampler.rs:75-87,filters.rs:37-43}
 * Built with -ffp-contract=off: every float operation is one IEEE operation
 * in the reference's order; fmaf() stands exactly where it calls mul_add.
 * expf/sinf/cosf/powf/sqrtf are glibc's, the functions Rust's std calls on
 * Linux.
 */
#include "rh_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

struct orc_decoder {
    orc_decoder_config c;
    orc_decoder_weights w;
    int threads;
    size_t kv_dim;
    float *keys, *values; /* [layer][context][kv_dim] */
    size_t *rows;         /* cached positions per layer */
};

static size_t mat_row_bytes(const orc_matrix *m)
{
    return m->type_id == 0 ? m->cols * 4 : orc_row_bytes(m->type_id, m->cols);
}

static orc_job mat_job(const orc_matrix *m, float *out, size_t out_len)
{
    orc_job j;
    memset(&j, 0, sizeof j);
    if (m->type_id == 0) {
        j.kind = ORC_DENSE;
        j.data_len = m->rows * m->cols;
        j.width = m->cols;
    } else {
        j.kind = m->type_id == 36 ? ORC_TERNARY : ORC_BLOCKS;
        j.type_id = m->type_id;
        j.width = mat_row_bytes(m);
        j.data_len = m->rows * j.width;
        /* Matrix::load (model/src/weights.rs:70-80): an I2_S matrix's scale
         * opens the trailer after its rows, which the caller passes along */
        if (m->type_id == 36)
            orc_i2s_scale((const uint8_t *)m->data + j.data_len, 32, &j.scale);
    }
    j.data = m->data;
    j.out = out;
    j.out_len = out_len;
    return j;
}

orc_decoder *orc_decoder_new(const orc_decoder_config *c, const orc_decoder_weights *w, int threads)
{
    orc_decoder *d = (orc_decoder *)calloc(1, sizeof *d);
    if (!d) return NULL;
    d->c = *c;
    d->w = *w;
    d->threads = threads > 0 ? threads : 1;
    d->kv_dim = c->head_count_kv * c->head_dim;
    size_t n = c->block_count * c->context_length * d->kv_dim;
    d->keys = (float *)calloc(n ? n : 1, sizeof(float));
    d->values = (float *)calloc(n ? n : 1, sizeof(float));
    d->rows = (size_t *)calloc(c->block_count ? c->block_count : 1, sizeof(size_t));
    if (!d->keys || !d->values || !d->rows) {
        orc_decoder_free(d);
        return NULL;
    }
    return d;
}

void orc_decoder_free(orc_decoder *d)
{
    if (!d) return;
    free(d->keys);
    free(d->values);
    free(d->rows);
    free(d);
}

/* KvCache::clear, model/src/cache.rs:79-83. */
void orc_decoder_reset(orc_decoder *d)
{
    memset(d->rows, 0, d->c.block_count * sizeof(size_t));
}

/* portable/norm.rs:8-14 then mul_assign: transformer/src/norm.rs:10-14. */
void orc_normalize(const float *in, const float *weight, size_t n, float eps, float *out)
{
    float sum = -0.0f;
    for (size_t i = 0; i < n; i++) {
        float sq = in[i] * in[i];
        sum += sq;
    }
    float mean_square = sum / (float)n;
    float rms = sqrtf(mean_square + eps);
    for (size_t i = 0; i < n; i++) {
        float v = in[i] / rms;
        out[i] = v * weight[i];
    }
}

/* portable/norm.rs:17-30: max from -inf, exp, sum from 0.0, divide. */
void orc_softmax(float *row, size_t n)
{
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, row[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        row[i] = expf(row[i] - max);
        sum += row[i];
    }
    for (size_t i = 0; i < n; i++) row[i] /= sum;
}

/* portable/rope.rs:7-23: pair p of `columns` rotated by position *
 * theta^(-2p/columns); low' = low*cos - high*sin (fused), high' = high*cos +
 * low*sin (fused). */
void orc_rope_adjacent(float *row, size_t len, size_t position, float theta, size_t dim_pairs)
{
    float columns = (float)len;
    float pos = (float)position;
    size_t pairs = len / 2 < dim_pairs ? len / 2 : dim_pairs;
    for (size_t p = 0; p < pairs; p++) {
        float exponent = -(float)(2 * p) / columns;
        float freq = powf(theta, exponent);
        float angle = pos * freq;
        float s = sinf(angle), c = cosf(angle);
        float lo = row[2 * p], hi = row[2 * p + 1];
        float hs = hi * s, ls = lo * s;
        row[2 * p] = fmaf(lo, c, -hs);
        row[2 * p + 1] = fmaf(hi, c, ls);
    }
}

/* The angle table RoPE reads: cos/sin of position * theta^(-2p/columns) for
 * every (position, pair), computed exactly as orc_rope_adjacent does. */
void orc_rope_table(size_t positions, size_t columns, float theta, float *cos_out, float *sin_out)
{
    size_t pairs = columns / 2;
    for (size_t pos = 0; pos < positions; pos++)
        for (size_t p = 0; p < pairs; p++) {
            float exponent = -(float)(2 * p) / (float)columns;
            float angle = (float)pos * powf(theta, exponent);
            cos_out[pos * pairs + p] = cosf(angle);
            sin_out[pos * pairs + p] = sinf(angle);
        }
}

/* f32::exp: libm's expf (what Rust's std calls on Linux), over an array. */
void orc_expf_array(const float *x, float *y, size_t n)
{
    for (size_t i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* portable/elementwise.rs:6-9: value / (1 + exp(-value)). */
static float silu(float v)
{
    float e = expf(-v);
    float den = 1.0f + e;
    return v / den;
}

void orc_silu_array(const float *x, float *y, size_t n)
{
    for (size_t i = 0; i < n; i++) y[i] = silu(x[i]);
}

/* rusticide-simd/src/float.rs:38-58 dot_rows: out[i] = dot(query,
 * rows_i[offset..offset+qlen]) / scale over nrows stride-wide rows (a zero
 * stride counts as one); a window past the row, or whose end overflows,
 * scores dot(query, []) / scale. */
void orc_dot_rows(const float *query, size_t qlen, const float *rows, size_t nrows, size_t stride, size_t offset,
                  float scale, float *out)
{
    if (stride == 0) stride = 1;
    const size_t end = offset + qlen;
    const int fits = end >= offset && end <= stride;
    for (size_t i = 0; i < nrows; i++) {
        const float *row = rows + i * stride;
        out[i] = (fits ? orc_dot_f32(query, qlen, row + offset, qlen) : orc_dot_f32(query, 0, row, 0)) / scale;
    }
}

/* float.rs:60-68 mix_rows: for rows i = 0.. in order, out[e] = fma(rows_i[offset
 * + e], weights[i], out[e]); min(nw, nrows) rows, windows past the row (or
 * whose end overflows) skipped, a zero stride counted as one. */
void orc_mix_rows(const float *weights, size_t nw, const float *rows, size_t nrows, size_t stride, size_t offset,
                  float *out, size_t n)
{
    if (stride == 0) stride = 1;
    const size_t end = offset + n;
    if (end < offset || end > stride) return;
    const size_t m = nw < nrows ? nw : nrows;
    for (size_t i = 0; i < m; i++)
        for (size_t e = 0; e < n; e++) out[e] = fmaf(rows[i * stride + offset + e], weights[i], out[e]);
}

/* layout.rs:9-27: out[row * tokens + token] -> one row per token. */
static void to_token_major(const float *by_row, size_t rows, size_t tokens, float *by_token)
{
    for (size_t t = 0; t < tokens; t++)
        for (size_t r = 0; r < rows; r++) by_token[t * rows + r] = by_row[r * tokens + t];
}

/* decoder.rs:111-136: one embedding row per token, after the context and
 * vocabulary checks. Returns 0 or an ORC_DEC_* error. */
static int embed(orc_decoder *d, const uint32_t *tokens, size_t n, size_t start, float *hidden)
{
    if (n == 0) return ORC_DEC_NO_TOKENS;
    if (start + n > d->c.context_length || start + n < start) return ORC_DEC_CONTEXT_FULL;
    const orc_matrix *e = &d->w.token_embd;
    size_t width = d->c.embedding_length, rb = mat_row_bytes(e);
    for (size_t t = 0; t < n; t++) {
        if (tokens[t] >= e->rows) return ORC_DEC_TOKEN_RANGE;
        const uint8_t *row = e->data + (size_t)tokens[t] * rb;
        if (e->type_id == 0) memcpy(hidden + t * width, row, width * 4);
        else orc_dequantize_row(e->type_id, row, rb, hidden + t * width, width);
    }
    return 0;
}

/* decoder.rs:74-107 (forward_batch): logits of the last token. */
int orc_decoder_forward_batch(orc_decoder *d, const uint32_t *tokens, size_t n, size_t start, float *logits)
{
    const orc_decoder_config *c = &d->c;
    size_t width = c->embedding_length, kv = d->kv_dim, ffn = c->feed_forward_length;
    size_t hd = c->head_dim, heads = c->head_count, group = c->head_count / c->head_count_kv;
    float scale = sqrtf((float)hd);
    float *hidden = (float *)malloc(n * width * 4), *normed = (float *)malloc(n * width * 4);
    float *delta = (float *)malloc(n * width * 4);
    float *qr = (float *)malloc(n * width * 4), *kr = (float *)malloc(n * kv * 4), *vr = (float *)malloc(n * kv * 4);
    float *q = (float *)malloc(n * width * 4), *k = (float *)malloc(n * kv * 4), *v = (float *)malloc(n * kv * 4);
    float *mixed = (float *)malloc(n * width * 4), *orows = (float *)malloc(n * width * 4);
    float *gate = (float *)malloc(n * ffn * 4), *up = (float *)malloc(n * ffn * 4), *hf = (float *)malloc(n * ffn * 4);
    float *scores = (float *)malloc((c->context_length + 1) * 4);
    int err = 0;
    if (!hidden || !normed || !delta || !qr || !kr || !vr || !q || !k || !v || !mixed || !orows || !gate || !up ||
        !hf || !scores) {
        err = ORC_DEC_NO_MEMORY;
        goto out;
    }
    if ((err = embed(d, tokens, n, start, hidden)) != 0) goto out;
    for (size_t layer = 0; layer < c->block_count; layer++) {
        const orc_block *b = &d->w.blocks[layer];
        for (size_t t = 0; t < n; t++)
            orc_normalize(hidden + t * width, b->attn_norm, width, c->rms_norm_eps, normed + t * width);
        /* attention.rs:210-230: Q/K/V in one batch, then token-major */
        orc_job jobs[3] = {mat_job(&b->attn_q, qr, n * width), mat_job(&b->attn_k, kr, n * kv),
                           mat_job(&b->attn_v, vr, n * kv)};
        orc_matmul_batch(normed, n * width, n, jobs, 3, d->threads);
        to_token_major(qr, width, n, q);
        to_token_major(kr, kv, n, k);
        to_token_major(vr, kv, n, v);
        /* attention.rs:156-183: rotate every head of q and k */
        for (size_t t = 0; t < n; t++) {
            for (size_t h = 0; h < heads; h++)
                orc_rope_adjacent(q + t * width + h * hd, hd, start + t, c->rope_freq_base, hd / 2);
            for (size_t h = 0; h < c->head_count_kv; h++)
                orc_rope_adjacent(k + t * kv + h * hd, hd, start + t, c->rope_freq_base, hd / 2);
        }
        /* cache.rs:35-65 */
        if (d->rows[layer] != start) {
            err = ORC_DEC_CACHE_POSITION;
            goto out;
        }
        float *kc = d->keys + layer * c->context_length * kv, *vc = d->values + layer * c->context_length * kv;
        memcpy(kc + start * kv, k, n * kv * 4);
        memcpy(vc + start * kv, v, n * kv * 4);
        d->rows[layer] = start + n;
        /* attention.rs:189-207 and :41-57: (token, head) over rows 0..=start+t */
        for (size_t t = 0; t < n; t++)
            for (size_t h = 0; h < heads; h++) {
                size_t rows = start + t + 1, off = (h / group) * hd;
                const float *qh = q + t * width + h * hd;
                orc_dot_rows(qh, hd, kc, rows, kv, off, scale, scores);
                orc_softmax(scores, rows);
                float *mh = mixed + t * width + h * hd;
                for (size_t e = 0; e < hd; e++) mh[e] = 0.0f;
                orc_mix_rows(scores, rows, vc, rows, kv, off, mh, hd);
            }
        orc_job oj = mat_job(&b->attn_output, orows, n * width);
        orc_matmul_batch(mixed, n * width, n, &oj, 1, d->threads);
        to_token_major(orows, width, n, delta);
        for (size_t i = 0; i < n * width; i++) hidden[i] += delta[i];
        /* feed_forward.rs:45-79 */
        for (size_t t = 0; t < n; t++)
            orc_normalize(hidden + t * width, b->ffn_norm, width, c->rms_norm_eps, normed + t * width);
        orc_job fj[2] = {mat_job(&b->ffn_gate, gate, n * ffn), mat_job(&b->ffn_up, up, n * ffn)};
        orc_matmul_batch(normed, n * width, n, fj, 2, d->threads);
        for (size_t i = 0; i < n * ffn; i++) {
            float s = silu(gate[i]);
            gate[i] = s * up[i];
        }
        to_token_major(gate, ffn, n, hf);
        orc_job dj = mat_job(&b->ffn_down, orows, n * width);
        orc_matmul_batch(hf, n * ffn, n, &dj, 1, d->threads);
        to_token_major(orows, width, n, delta);
        for (size_t i = 0; i < n * width; i++) hidden[i] += delta[i];
    }
    /* decoder.rs:96-106: the last token's final norm and the output matvec */
    orc_normalize(hidden + (n - 1) * width, d->w.output_norm, width, c->rms_norm_eps, normed);
    {
        const orc_matrix *out = d->w.output ? d->w.output : &d->w.token_embd;
        orc_job lj = mat_job(out, logits, c->vocab_size);
        orc_matmul_batch(normed, width, 1, &lj, 1, d->threads);
    }
out:
    free(hidden); free(normed); free(delta); free(qr); free(kr); free(vr); free(q); free(k); free(v);
    free(mixed); free(orows); free(gate); free(up); free(hf); free(scores);
    return err;
}

/* f32::total_cmp's key: a sign-magnitude total order as i32. */
static int32_t total_key(float f)
{
    int32_t b;
    memcpy(&b, &f, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* Sampler::greedy_logits, sampling/src/sampler.rs:75-87 with argmax,
 * filters.rs:37-43: NaN counts as -inf; max_by keeps the last maximum. */
int orc_greedy(const float *logits, size_t n, uint32_t *token)
{
    int any_finite = 0;
    size_t best = 0;
    int32_t best_key = 0;
    for (size_t i = 0; i < n; i++) {
        float v = isnan(logits[i]) ? -INFINITY : logits[i];
        if (isfinite(logits[i])) any_finite = 1;
        int32_t key = total_key(v);
        if (i == 0 || key >= best_key) {
            best = i;
            best_key = key;
        }
    }
    if (n == 0 || !any_finite) return ORC_DEC_NO_VALID_TOKENS;
    *token = (uint32_t)best;
    return 0;
}

/* generate.rs:35-124 with temperature 0: reset, prefill in chunks of 64,
 * then pick / forward until max_tokens or the context end (no tokenizer, so
 * no end-of-generation token). */
int orc_generate_greedy(orc_decoder *d, const uint32_t *prompt, size_t n, size_t max_tokens, uint32_t *out,
                        size_t *n_out)
{
    *n_out = 0;
    if (n >= d->c.context_length) return ORC_DEC_CONTEXT_FULL;
    if (n == 0) return ORC_DEC_NO_TOKENS;
    float *logits = (float *)malloc(d->c.vocab_size * 4);
    if (!logits) return ORC_DEC_NO_MEMORY;
    orc_decoder_reset(d);
    int err = 0;
    for (size_t s = 0; s < n; s += 64) {
        size_t m = n - s < 64 ? n - s : 64;
        if ((err = orc_decoder_forward_batch(d, prompt + s, m, s, logits)) != 0) goto done;
    }
    size_t position = n;
    for (size_t i = 0; i < max_tokens; i++) {
        uint32_t next;
        if ((err = orc_greedy(logits, d->c.vocab_size, &next)) != 0) goto done;
        out[(*n_out)++] = next;
        if (position == d->c.context_length) break;
        if ((err = orc_decoder_forward_batch(d, &next, 1, position, logits)) != 0) goto done;
        position++;
    }
done:
    free(logits);
    return err;
}
