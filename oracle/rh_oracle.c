/*
 * rh_oracle.c -- CPU restatement of rusticide's quantized matrix-product
 * arithmetic (Q4_K / Q6_K x Q8_K integer dots, I2_S x I8_S ternary dots,
 * the f32 dot, the activation quantizers and the matmul_batch scheduler).
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker the HIP path is compared
 * against and the CPU baseline timed beside it; the product never links it.
 *
 * Written from the reference's source, read as text; paths are relative to
 * the rusticide repository root. Build with -ffp-contract=off and without
 * -ffast-math: every float operation below is one IEEE operation in the order
 * the reference performs it, and fmaf() appears exactly where the reference
 * calls mul_add.
 */
#include "rh_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#define Q8_BLOCK 32

/* ---------------------------------------------------------------- formats */

/* The block-format table, format.rs:31-92 (Q4_0/Q5_0/Q8_0 are out of scope). */
int orc_block_format(uint32_t type_id, size_t *block_size, size_t *block_bytes,
                     size_t *trailer_bytes)
{
    size_t bs, bb, tb;
    switch (type_id) {
    case 12: bs = 256; bb = 144; tb = 0; break;  /* Q4_K, q4_k.rs:10-11 */
    case 14: bs = 256; bb = 210; tb = 0; break;  /* Q6_K, q6_k.rs:10-11 */
    case 36: bs = 128; bb = 32; tb = 32; break;  /* I2_S, i2_s.rs:8-10  */
    default: return 0;
    }
    if (block_size) *block_size = bs;
    if (block_bytes) *block_bytes = bb;
    if (trailer_bytes) *trailer_bytes = tb;
    return 1;
}

/* format.rs:151-165: whole blocks rounded up, then the trailer. */
size_t orc_byte_len(uint32_t type_id, size_t numel)
{
    size_t bs, bb, tb;
    if (!orc_block_format(type_id, &bs, &bb, &tb)) return SIZE_MAX;
    size_t blocks = numel / bs + (numel % bs != 0);
    if (blocks > (SIZE_MAX - tb) / bb) return SIZE_MAX;
    return blocks * bb + tb;
}

/* format.rs:193-198: None unless cols is a whole number of blocks. */
size_t orc_row_bytes(uint32_t type_id, size_t cols)
{
    size_t bs, bb, tb;
    if (!orc_block_format(type_id, &bs, &bb, &tb)) return SIZE_MAX;
    if (cols % bs != 0) return SIZE_MAX;
    if (cols / bs > SIZE_MAX / bb) return SIZE_MAX;
    return cols / bs * bb;
}

/* ------------------------------------------------------------------- f16 */

/* IEEE binary16 -> binary32, exact (half_bits.rs:16-18; the scalar twin in
 * rusticide-simd/src/scalar.rs:19-34). NaN comes back quiet. */
float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man ? (0x00400000u | (man << 13)) : 0);
    } else if (exp == 0) {
        float v = ldexpf((float)man, -24); /* exact: man < 2^10 */
        return sign ? -v : v;
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even (half 2.7.1 f16::from_f32). */
uint16_t orc_f32_to_f16(float value)
{
    uint32_t x;
    memcpy(&x, &value, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0));
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        unsigned shift = (unsigned)(14 - e);
        uint32_t half_man = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_man & 1u))) half_man++;
        return (uint16_t)(sign | half_man);
    }
    uint32_t half = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
    return (uint16_t)half;
}

static float f16_at(const uint8_t *p)
{
    return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* ------------------------------------------------------------- dequantize */

/* ggml get_scale_min_k4, q4_k.rs:17-25. */
static void q4k_scale_min(int j, const uint8_t *s, uint8_t *sc, uint8_t *m)
{
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* q4_k.rs:32-66: d*sc*q - dmin*m, never fused (q4_k.rs:27-31). */
static void dequant_q4k(const uint8_t *b, float *out)
{
    float d = f16_at(b), dmin = f16_at(b + 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    for (int pair = 0; pair < 4; pair++) {
        uint8_t sl, ml, sh, mh;
        q4k_scale_min(2 * pair, scales, &sl, &ml);
        q4k_scale_min(2 * pair + 1, scales, &sh, &mh);
        float dl = d * (float)sl, ml_f = dmin * (float)ml;
        float dh = d * (float)sh, mh_f = dmin * (float)mh;
        for (int l = 0; l < 32; l++) {
            uint8_t q = qs[32 * pair + l];
            volatile float lo = dl * (float)(q & 0x0f);
            volatile float hi = dh * (float)(q >> 4);
            out[64 * pair + l] = lo - ml_f;
            out[64 * pair + 32 + l] = hi - mh_f;
        }
    }
}

/* q6_k.rs:13-43. */
static float six_bit_f(uint8_t low, uint8_t high)
{
    return (float)((int)(low | ((high & 3) << 4)) - 32);
}

static void dequant_q6k(const uint8_t *b, float *out)
{
    float d = f16_at(b + 208);
    for (int h = 0; h < 2; h++) {
        const uint8_t *low = b + 64 * h, *high = b + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * h);
        float *o = out + 128 * h;
        for (int l = 0; l < 32; l++) {
            int g = l / 16;
            float q1 = six_bit_f(low[l] & 0x0f, high[l]);
            float q2 = six_bit_f(low[l + 32] & 0x0f, high[l] >> 2);
            float q3 = six_bit_f(low[l] >> 4, high[l] >> 4);
            float q4 = six_bit_f(low[l + 32] >> 4, high[l] >> 6);
            volatile float t;
            t = d * (float)sc[g + 0]; o[l] = t * q1;
            t = d * (float)sc[g + 2]; o[l + 32] = t * q2;
            t = d * (float)sc[g + 4]; o[l + 64] = t * q3;
            t = d * (float)sc[g + 6]; o[l + 96] = t * q4;
        }
    }
}

/* i2_s.rs:12-21: byte k holds weights k, k+32, k+64, k+96 at shifts 6,4,2,0;
 * code c decodes to c - 1 (code 3 to +2). */
static void dequant_i2s(const uint8_t *b, float *out)
{
    static const int shifts[4] = {6, 4, 2, 0};
    for (int lane = 0; lane < 4; lane++)
        for (int k = 0; k < 32; k++)
            out[32 * lane + k] = (float)((b[k] >> shifts[lane]) & 3) - 1.0f;
}

/* format.rs:219-226: whole blocks of the row, bounded by the shorter side. */
void orc_dequantize_row(uint32_t type_id, const uint8_t *row, size_t row_len,
                        float *out, size_t out_len)
{
    size_t bs, bb;
    if (!orc_block_format(type_id, &bs, &bb, NULL)) return;
    size_t n = row_len / bb;
    if (out_len / bs < n) n = out_len / bs;
    for (size_t i = 0; i < n; i++) {
        if (type_id == 12) dequant_q4k(row + i * bb, out + i * bs);
        else if (type_id == 14) dequant_q6k(row + i * bb, out + i * bs);
        else dequant_i2s(row + i * bb, out + i * bs);
    }
}

/* i2_s.rs:26-30. */
int orc_i2s_scale(const uint8_t *trailer, size_t len, float *scale)
{
    if (len < 4) return 0;
    memcpy(scale, trailer, 4); /* little-endian host */
    return 1;
}

/* -------------------------------------------------------------- generators */

/* format.rs:109-117: the top byte of a 32-bit LCG. */
void orc_pseudo_random_bytes(uint8_t *out, size_t len, uint32_t seed)
{
    uint32_t state = seed;
    for (size_t i = 0; i < len; i++) {
        state = state * 1664525u + 1013904223u;
        out[i] = (uint8_t)(state >> 24);
    }
}

/* format.rs:106,204-214: random bytes, then every f16 scale field set to one
 * of 0.01..0.07 in turn. */
int orc_synthetic_blocks(uint32_t type_id, size_t blocks, uint32_t seed, uint8_t *out)
{
    static const float SCALES[7] = {0.01f, 0.02f, 0.03f, 0.04f, 0.05f, 0.06f, 0.07f};
    size_t bs, bb;
    if (!orc_block_format(type_id, &bs, &bb, NULL)) return 0;
    orc_pseudo_random_bytes(out, blocks * bb, seed);
    size_t offsets[2];
    size_t n_off = 0;
    if (type_id == 12) { offsets[0] = 0; offsets[1] = 2; n_off = 2; }
    if (type_id == 14) { offsets[0] = 208; n_off = 1; }
    for (size_t i = 0; i < blocks; i++) {
        uint16_t h = orc_f32_to_f16(SCALES[i % 7]);
        for (size_t k = 0; k < n_off; k++) {
            out[i * bb + offsets[k]] = (uint8_t)(h & 0xff);
            out[i * bb + offsets[k] + 1] = (uint8_t)(h >> 8);
        }
    }
    return 1;
}

/* kernels/src/test_support.rs:72-80: values in [-1, 1). */
void orc_pseudo_random_values(float *out, size_t len, uint32_t seed)
{
    uint32_t state = seed;
    for (size_t i = 0; i < len; i++) {
        state = state * 1664525u + 1013904223u;
        out[i] = (float)(state >> 24) / 128.0f - 1.0f;
    }
}

/* bench/src/kernels.rs:27-35. */
void orc_bench_activations(float *out, size_t len, uint32_t seed)
{
    uint32_t state = seed;
    for (size_t i = 0; i < len; i++) {
        state = state * 1664525u + 1013904223u;
        out[i] = (float)(uint16_t)(state >> 16) / 32768.0f - 1.0f;
    }
}

/* -------------------------------------------------------------- quantizers */

/* round_to_i8, portable/q8.rs:114-116: ties to even, clamp to +-127, NaN
 * (which clamp keeps) casts to 0. */
static int8_t round_to_i8(float v)
{
    float r = rintf(v);
    if (r != r) return 0;
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)r;
}

/* round_row_to_i8, portable/q8.rs:128-130: ties to even then Rust's
 * saturating `as i8` (NaN -> 0, beyond the range -> the bound). */
static int8_t round_row_to_i8(float v)
{
    float r = rintf(v);
    if (r != r) return 0;
    if (r <= -128.0f) return -128;
    if (r >= 127.0f) return 127;
    return (int8_t)r;
}

/* f32::max: a NaN operand yields the other one (IEEE maxNum). */
static float rust_max(float a, float b)
{
    return fmaxf(a, b);
}

/* portable/q8.rs:64-106. */
size_t orc_quantize(int kind, const float *x, size_t len, int8_t *quants,
                    float *scales, int32_t *sums)
{
    size_t n_blocks = len / Q8_BLOCK;
    if (kind == ORC_Q8_SUPER_BLOCK) {
        n_blocks = n_blocks / 8 * 8;
        for (size_t sb = 0; sb < n_blocks / 8; sb++) {
            const float *v = x + sb * 256;
            /* signed_max, q8.rs:19-33: amax per block, folded from 0.0 */
            float amax = 0.0f;
            for (int b = 0; b < 8; b++) {
                float block_max = 0.0f;
                for (int i = 0; i < 32; i++) block_max = rust_max(block_max, fabsf(v[32 * b + i]));
                amax = rust_max(amax, block_max);
            }
            float max = 0.0f;
            for (int i = 0; i < 256; i++) {
                if (fabsf(v[i]) == amax) { max = v[i]; break; }
            }
            float inverse = (max == 0.0f) ? 0.0f : -127.0f / max;
            float step = (max == 0.0f) ? 0.0f : 1.0f / inverse;
            for (int b = 0; b < 8; b++) {
                int32_t sum = 0;
                for (int i = 0; i < 32; i++) {
                    int8_t q = round_to_i8(v[32 * b + i] * inverse);
                    quants[sb * 256 + 32 * b + i] = q;
                    sum += q;
                }
                sums[sb * 8 + b] = sum;
                scales[sb * 8 + b] = step;
            }
        }
        return n_blocks;
    }
    if (kind == ORC_Q8_ROW) {
        /* row_divisor, q8.rs:38-49: C's MAX macro in f64 from 1e-5. */
        double mx = 1e-5;
        for (size_t i = 0; i < n_blocks * Q8_BLOCK; i++) {
            double mag = (double)fabsf(x[i]);
            mx = (mx > mag) ? mx : mag;
        }
        float divisor = (float)(127.0 / mx);
        for (size_t b = 0; b < n_blocks; b++) {
            int32_t sum = 0;
            for (int i = 0; i < 32; i++) {
                int8_t q = round_row_to_i8(x[b * 32 + i] * divisor);
                quants[b * 32 + i] = q;
                sum += q;
            }
            sums[b] = sum;
            scales[b] = divisor;
        }
        return n_blocks;
    }
    return 0;
}

/* q8_input.rs:72-93: scale * q, or q / scale for Row. */
void orc_q8_dequantize(int kind, const int8_t *quants, const float *scales,
                       size_t n_blocks, float *out)
{
    for (size_t b = 0; b < n_blocks; b++)
        for (int i = 0; i < 32; i++)
            out[b * 32 + i] = (kind == ORC_Q8_ROW) ? (float)quants[b * 32 + i] / scales[b]
                                                   : scales[b] * (float)quants[b * 32 + i];
}

/* ---------------------------------------------------------- integer dots */

/* k4_scales_and_mins, portable/int_dot.rs:126-140 (same values as
 * q4k_scale_min, unpacked a word at a time as ggml does). */
static void k4_scales_and_mins(const uint8_t *p, uint8_t sc[8], uint8_t mn[8])
{
    uint32_t first = p[0] | p[1] << 8 | p[2] << 16 | (uint32_t)p[3] << 24;
    uint32_t second = p[4] | p[5] << 8 | p[6] << 16 | (uint32_t)p[7] << 24;
    uint32_t third = p[8] | p[9] << 8 | p[10] << 16 | (uint32_t)p[11] << 24;
    uint32_t hs = (third & 0x0f0f0f0fu) | (((first >> 6) & 0x03030303u) << 4);
    uint32_t hm = ((third >> 4) & 0x0f0f0f0fu) | (((second >> 6) & 0x03030303u) << 4);
    uint32_t ls = first & 0x3f3f3f3fu, lm = second & 0x3f3f3f3fu;
    for (int i = 0; i < 4; i++) {
        sc[i] = (uint8_t)(ls >> (8 * i));
        sc[i + 4] = (uint8_t)(hs >> (8 * i));
        mn[i] = (uint8_t)(lm >> (8 * i));
        mn[i + 4] = (uint8_t)(hm >> (8 * i));
    }
}

/* One Q4_K block against one span of eight Q8_K blocks, int_dot.rs:146-170:
 * term = d8 * fma(d, isum, -(dmin * msum)). */
static float q4k_block_term(const uint8_t *b, const int8_t *q, const float *scales,
                            const int32_t *sums)
{
    uint8_t sc[8], mn[8];
    k4_scales_and_mins(b + 4, sc, mn);
    int32_t sum = 0;
    for (int pair = 0; pair < 4; pair++) {
        const uint8_t *packed = b + 16 + 32 * pair;
        const int8_t *lq = q + 64 * pair, *hq = q + 64 * pair + 32;
        int32_t low = 0, high = 0;
        for (int l = 0; l < 32; l++) {
            low += ((int)(packed[l] & 0x0f) - 8) * lq[l];
            high += ((int)(packed[l] >> 4) - 8) * hq[l];
        }
        sum += (int32_t)sc[2 * pair] * low;
        sum += (int32_t)sc[2 * pair + 1] * high;
    }
    int32_t min_sum = 0;
    for (int j = 0; j < 8; j++) {
        sum += 8 * (int32_t)sc[j] * sums[j];
        min_sum += (int32_t)mn[j] * sums[j];
    }
    float d = f16_at(b), dmin = f16_at(b + 2);
    float neg = -(dmin * (float)min_sum);
    return scales[0] * fmaf(d, (float)sum, neg);
}

/* One Q6_K block, int_dot.rs:182-203: term = (d * d8) * isum. */
static float q6k_block_term(const uint8_t *b, const int8_t *q, const float *scales)
{
    int32_t sum = 0;
    for (int half = 0; half < 2; half++) {
        const uint8_t *low = b + 64 * half, *high = b + 128 + 32 * half;
        const uint8_t *sc = b + 192 + 8 * half;
        const int8_t *hq = q + 128 * half;
        for (int group = 0; group < 2; group++) {
            int32_t runs[4] = {0, 0, 0, 0};
            for (int l = 16 * group; l < 16 * (group + 1); l++) {
                uint8_t first = low[l], second = low[l + 32], bits = high[l];
                runs[0] += ((int)((first & 0x0f) | (((bits >> 0) & 3) << 4)) - 32) * hq[l];
                runs[1] += ((int)((second & 0x0f) | (((bits >> 2) & 3) << 4)) - 32) * hq[32 + l];
                runs[2] += ((int)((first >> 4) | (((bits >> 4) & 3) << 4)) - 32) * hq[64 + l];
                runs[3] += ((int)((second >> 4) | (((bits >> 6) & 3) << 4)) - 32) * hq[96 + l];
            }
            for (int run = 0; run < 4; run++) sum += (int32_t)(int8_t)sc[2 * run + group] * runs[run];
        }
    }
    float d = f16_at(b + 208);
    float dd = d * scales[0];
    return dd * (float)sum;
}

/* dot_row, int_dot.rs:36-47: block terms summed in row order from -0.0 over
 * the blocks both operands cover. */
float orc_q4k_dot(const uint8_t *row, size_t row_len, const int8_t *quants,
                  const float *scales, const int32_t *sums, size_t n_blocks)
{
    size_t n = row_len / 144;
    if (n_blocks / 8 < n) n = n_blocks / 8;
    float acc = -0.0f;
    for (size_t i = 0; i < n; i++)
        acc += q4k_block_term(row + 144 * i, quants + 256 * i, scales + 8 * i, sums + 8 * i);
    return acc;
}

float orc_q6k_dot(const uint8_t *row, size_t row_len, const int8_t *quants,
                  const float *scales, const int32_t *sums, size_t n_blocks)
{
    (void)sums;
    size_t n = row_len / 210;
    if (n_blocks / 8 < n) n = n_blocks / 8;
    float acc = -0.0f;
    for (size_t i = 0; i < n; i++)
        acc += q6k_block_term(row + 210 * i, quants + 256 * i, scales + 8 * i);
    return acc;
}

/* ternary_dot, portable/ternary.rs:21-42: per block sum(code*q) - sum(q),
 * blocks folded with wrapping i32 addition. */
int32_t orc_ternary_dot(const uint8_t *row, size_t row_len, const int8_t *quants,
                        const int32_t *sums, size_t n_blocks)
{
    static const int shifts[4] = {6, 4, 2, 0};
    size_t n = row_len / 32;
    if (n_blocks / 4 < n) n = n_blocks / 4;
    uint32_t acc = 0;
    for (size_t i = 0; i < n; i++) {
        const uint8_t *b = row + 32 * i;
        int32_t products = 0;
        for (int lane = 0; lane < 4; lane++) {
            int32_t s = 0;
            for (int k = 0; k < 32; k++)
                s += (int32_t)((b[k] >> shifts[lane]) & 3) * quants[128 * i + 32 * lane + k];
            products += s;
        }
        int32_t q_sum = sums[4 * i] + sums[4 * i + 1] + sums[4 * i + 2] + sums[4 * i + 3];
        acc += (uint32_t)(products - q_sum);
    }
    return (int32_t)acc;
}

/* product, portable/ternary.rs:48-58: (dot / s) * scale, 0 without a scale. */
float orc_ternary_product(const uint8_t *row, size_t row_len, const int8_t *quants,
                          const float *scales, const int32_t *sums, size_t n_blocks,
                          float scale)
{
    float dot = (float)orc_ternary_dot(row, row_len, quants, sums, n_blocks);
    if (n_blocks == 0) return 0.0f;
    float t = dot / scales[0];
    return t * scale;
}

/* rusticide-simd/src/float.rs:23-36: eight fused lanes, then the lanes summed
 * in order from -0.0, then the unfused tail summed from -0.0. */
float orc_dot_f32(const float *lhs, size_t lhs_len, const float *rhs, size_t rhs_len)
{
    size_t n = lhs_len < rhs_len ? lhs_len : rhs_len;
    size_t chunks = n / 8;
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t c = 0; c < chunks; c++)
        for (int i = 0; i < 8; i++) lanes[i] = fmaf(lhs[8 * c + i], rhs[8 * c + i], lanes[i]);
    float tail = -0.0f;
    for (size_t i = 8 * chunks; i < n; i++) {
        volatile float p = lhs[i] * rhs[i];
        tail += p;
    }
    float sum = -0.0f;
    for (int i = 0; i < 8; i++) sum += lanes[i];
    return sum + tail;
}

/* quant_kernel_tests.rs:29-31: the dequantized row against activation values,
 * products summed in order from -0.0. */
float orc_dequant_dot(uint32_t type_id, const uint8_t *row, size_t row_len,
                      const float *x, size_t x_len)
{
    size_t bs, bb;
    if (!orc_block_format(type_id, &bs, &bb, NULL)) return 0.0f;
    size_t n = row_len / bb * bs;
    float *w = (float *)malloc(n * sizeof(float) + 1);
    orc_dequantize_row(type_id, row, row_len, w, n);
    size_t m = n < x_len ? n : x_len;
    float acc = -0.0f;
    for (size_t i = 0; i < m; i++) {
        volatile float p = w[i] * x[i];
        acc += p;
    }
    free(w);
    return acc;
}

/* ------------------------------------------------------------ matmul_batch */

typedef struct {
    size_t n_blocks;
    int8_t *quants;
    float *scales;
    int32_t *sums;
} q8_input;

typedef struct {
    const orc_job *job;
    size_t first_row, n_rows;
} run_t;

typedef struct {
    const float *inputs;
    size_t width, tokens;
    q8_input *super_block, *row;
    run_t *runs;
    size_t n_runs;
    atomic_size_t next;
} batch_t;

static size_t job_rows(const orc_job *job)
{
    return job->width ? job->data_len / job->width : 0;
}

/* Weights::compute_rows, matmul.rs:93-128, for rows first..first+n. */
static void compute_run(batch_t *b, const run_t *r)
{
    const orc_job *job = r->job;
    size_t tokens = b->tokens;
    for (size_t row = r->first_row; row < r->first_row + r->n_rows; row++) {
        for (size_t t = 0; t < tokens; t++) {
            size_t idx = row * tokens + t;
            if (idx >= job->out_len) return;
            float v;
            if (job->kind == ORC_DENSE) {
                const float *w = (const float *)job->data + row * job->width;
                v = orc_dot_f32(w, job->width, b->inputs + t * b->width, b->width);
            } else if (job->kind == ORC_TERNARY) {
                const uint8_t *w = (const uint8_t *)job->data + row * job->width;
                q8_input *in = &b->row[t];
                v = orc_ternary_product(w, job->width, in->quants, in->scales, in->sums,
                                        in->n_blocks, job->scale);
            } else {
                const uint8_t *w = (const uint8_t *)job->data + row * job->width;
                q8_input *in = &b->super_block[t];
                v = job->type_id == 12
                        ? orc_q4k_dot(w, job->width, in->quants, in->scales, in->sums, in->n_blocks)
                        : orc_q6k_dot(w, job->width, in->quants, in->scales, in->sums, in->n_blocks);
            }
            job->out[idx] = v;
        }
    }
}

static void *worker(void *arg)
{
    batch_t *b = (batch_t *)arg;
    for (;;) {
        size_t i = atomic_fetch_add(&b->next, 1);
        if (i >= b->n_runs) break;
        compute_run(b, &b->runs[i]);
    }
    return NULL;
}

static q8_input *quantize_tokens(int kind, const float *inputs, size_t width, size_t tokens)
{
    q8_input *qs = (q8_input *)calloc(tokens, sizeof(q8_input));
    for (size_t t = 0; t < tokens; t++) {
        size_t nb = width / 32 + 1;
        qs[t].quants = (int8_t *)malloc(nb * 32);
        qs[t].scales = (float *)malloc(nb * sizeof(float));
        qs[t].sums = (int32_t *)malloc(nb * sizeof(int32_t));
        qs[t].n_blocks = orc_quantize(kind, inputs + t * width, width, qs[t].quants,
                                      qs[t].scales, qs[t].sums);
    }
    return qs;
}

static void free_tokens(q8_input *qs, size_t tokens)
{
    if (!qs) return;
    for (size_t t = 0; t < tokens; t++) {
        free(qs[t].quants);
        free(qs[t].scales);
        free(qs[t].sums);
    }
    free(qs);
}

/* matmul.rs:229-248: quantize each activation kind once per token, split the
 * rows into threads*16 runs, compute them in parallel. */
void orc_matmul_batch(const float *inputs, size_t inputs_len, size_t tokens,
                      const orc_job *jobs, size_t n_jobs, int threads)
{
    if (tokens == 0 || tokens > inputs_len) return;
    if (threads <= 0) threads = 1;
    batch_t b;
    memset(&b, 0, sizeof(b));
    b.inputs = inputs;
    b.width = inputs_len / tokens;
    b.tokens = tokens;
    int want_super = 0, want_row = 0;
    size_t total = 0;
    for (size_t j = 0; j < n_jobs; j++) {
        if (jobs[j].kind == ORC_BLOCKS) want_super = 1;
        if (jobs[j].kind == ORC_TERNARY) want_row = 1;
        total += job_rows(&jobs[j]);
    }
    if (want_super) b.super_block = quantize_tokens(ORC_Q8_SUPER_BLOCK, inputs, b.width, tokens);
    if (want_row) b.row = quantize_tokens(ORC_Q8_ROW, inputs, b.width, tokens);
    size_t tasks = (size_t)threads * 16;
    size_t rows_per_task = (total + tasks - 1) / tasks;
    if (rows_per_task == 0) rows_per_task = 1;
    size_t cap = tasks + n_jobs + 1;
    b.runs = (run_t *)malloc(cap * sizeof(run_t));
    for (size_t j = 0; j < n_jobs; j++) {
        size_t rows = job_rows(&jobs[j]);
        for (size_t first = 0; first < rows; first += rows_per_task) {
            if (b.n_runs == cap) {
                cap *= 2;
                b.runs = (run_t *)realloc(b.runs, cap * sizeof(run_t));
            }
            size_t n = rows - first < rows_per_task ? rows - first : rows_per_task;
            b.runs[b.n_runs++] = (run_t){&jobs[j], first, n};
        }
    }
    atomic_init(&b.next, 0);
    if (threads == 1) {
        worker(&b);
    } else {
        pthread_t *ids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
        for (int i = 0; i < threads; i++) pthread_create(&ids[i], NULL, worker, &b);
        for (int i = 0; i < threads; i++) pthread_join(ids[i], NULL);
        free(ids);
    }
    free(b.runs);
    free_tokens(b.super_block, tokens);
    free_tokens(b.row, tokens);
}

void orc_ternary_dot_matrix_i32(const uint8_t *data, size_t data_len, size_t row_bytes,
                                const float *inputs, size_t inputs_len, size_t tokens,
                                int32_t *out, size_t out_len)
{
    if (tokens == 0 || tokens > inputs_len || row_bytes == 0) return;
    size_t width = inputs_len / tokens;
    q8_input *in = quantize_tokens(ORC_Q8_ROW, inputs, width, tokens);
    size_t rows = data_len / row_bytes;
    for (size_t r = 0; r < rows; r++)
        for (size_t t = 0; t < tokens; t++) {
            size_t idx = r * tokens + t;
            if (idx >= out_len) goto done;
            out[idx] = orc_ternary_dot(data + r * row_bytes, row_bytes, in[t].quants,
                                       in[t].sums, in[t].n_blocks);
        }
done:
    free_tokens(in, tokens);
}
