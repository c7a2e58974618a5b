/*
 * tnref -- CPU oracle (TEST INFRASTRUCTURE ONLY; see tnref.h).
 *
 * Build with -O2 -ffp-contract=off and no fast-math at the baseline x86-64 ISA:
 * Rust never contracts a*b+c into an FMA and the reference's x86_64 wheel sets
 * no target-cpu, so every float operation below must round on its own.
 */
#include "tnref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QK 32

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* Reduced floats                                                           */
/* ------------------------------------------------------------------------ */

/* f32 -> f16, round to nearest even, subnormals kept, overflow to inf.
 * This is the IEEE conversion half 2.7.1's `f16::from_f32` performs (the
 * reference's Cargo.lock pins half 2.7.1; BlockQ4_0/BlockQ8_0 store `d` with
 * it, K:263 and K:700). NaN keeps its sign and top payload bits, quieted. */
uint16_t tnref_f16_from_f32(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7c00u | 0x0200u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* subnormal half (or zero): shift the full significand down */
        if (14 - e > 24) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t hm = m >> shift;
        uint32_t round_bit = 1u << (shift - 1);
        if ((m & round_bit) && (m & (3u * round_bit - 1u))) hm += 1;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t round_bit = 0x1000u;
    if ((man & round_bit) && (man & (3u * round_bit - 1u))) h += 1; /* may carry into exp: correct */
    return (uint16_t)h;
}

float tnref_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    if (exp == 0x1fu) return bits_f32(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: value = man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

/* f32 -> bf16, round to nearest even, NaN quieted (R:161-218). */
uint16_t tnref_bf16_from_f32(float f) {
    uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

float tnref_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

void tnref_f32_to_f16_n(const float* s, uint16_t* d, int64_t n) {
    for (int64_t i = 0; i < n; i++) d[i] = tnref_f16_from_f32(s[i]);
}
void tnref_f32_to_bf16_n(const float* s, uint16_t* d, int64_t n) {
    for (int64_t i = 0; i < n; i++) d[i] = tnref_bf16_from_f32(s[i]);
}
void tnref_bf16_to_f32_n(const uint16_t* s, float* d, int64_t n) {
    for (int64_t i = 0; i < n; i++) d[i] = tnref_bf16_to_f32(s[i]);
}

/* ------------------------------------------------------------------------ */
/* Rust cast semantics                                                       */
/* ------------------------------------------------------------------------ */

/* `f as u8`: truncate toward zero, saturate to [0, 255], NaN -> 0. */
static inline uint8_t as_u8(float v) {
    if (v != v) return 0;
    if (v >= 255.0f) return 255;
    if (v <= 0.0f) return 0;
    return (uint8_t)v;
}

/* `f as i8`: truncate toward zero, saturate to [-128, 127], NaN -> 0. */
static inline int8_t as_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* ------------------------------------------------------------------------ */
/* Q4_0 / Q8_0 codecs                                                        */
/* ------------------------------------------------------------------------ */

/* BlockQ4_0::from_float, K:241-277. Signed extreme kept: d = max / -8. */
void tnref_q4_0_quantize(const float* x, int64_t n, uint8_t* blob) {
    for (int64_t b = 0; b < n / QK; b++) {
        const float* xs = x + b * QK;
        uint8_t* out = blob + b * 18;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < QK; j++) {
            float a = fabsf(xs[j]);
            if (amax < a) { amax = a; mx = xs[j]; }
        }
        float d = mx / -8.0f;
        float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        uint16_t h = tnref_f16_from_f32(d);
        out[0] = (uint8_t)(h & 0xff);
        out[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < QK / 2; j++) {
            float x0 = xs[j] * id;
            float x1 = xs[QK / 2 + j] * id;
            uint8_t q0 = as_u8(x0 + 8.5f);
            uint8_t q1 = as_u8(x1 + 8.5f);
            if (q0 > 15) q0 = 15;
            if (q1 > 15) q1 = 15;
            out[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

/* BlockQ4_0::to_float, K:219-239: (nib - 8) as f32 * f32(d). */
void tnref_q4_0_dequantize(const uint8_t* blob, int64_t n, float* y) {
    for (int64_t b = 0; b < n / QK; b++) {
        const uint8_t* in = blob + b * 18;
        float d = tnref_f16_to_f32((uint16_t)(in[0] | (in[1] << 8)));
        for (int j = 0; j < QK / 2; j++) {
            int x0 = (in[2 + j] & 0x0f) - 8;
            int x1 = (in[2 + j] >> 4) - 8;
            y[b * QK + j] = (float)x0 * d;
            y[b * QK + j + QK / 2] = (float)x1 * d;
        }
    }
}

/* BlockQ8_0::from_float, K:676-705. `id` uses the f32 d, not the f16 one;
 * f32::max ignores a NaN operand, as fmaxf does; f32::round is half away
 * from zero, as roundf is. */
void tnref_q8_0_quantize(const float* x, int64_t n, uint8_t* blob) {
    for (int64_t b = 0; b < n / QK; b++) {
        const float* xs = x + b * QK;
        uint8_t* out = blob + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(xs[j]));
        float d = amax / 127.0f;
        float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        uint16_t h = tnref_f16_from_f32(d);
        out[0] = (uint8_t)(h & 0xff);
        out[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < QK; j++) out[2 + j] = (uint8_t)as_i8(roundf(xs[j] * id));
    }
}

/* BlockQ8_0::to_float, K:659-674. */
void tnref_q8_0_dequantize(const uint8_t* blob, int64_t n, float* y) {
    for (int64_t b = 0; b < n / QK; b++) {
        const uint8_t* in = blob + b * 34;
        float d = tnref_f16_to_f32((uint16_t)(in[0] | (in[1] << 8)));
        for (int j = 0; j < QK; j++) y[b * QK + j] = (float)(int8_t)in[2 + j] * d;
    }
}

/* ------------------------------------------------------------------------ */
/* The quantised linear                                                      */
/* ------------------------------------------------------------------------ */

/* BlockQ4_0::vec_dot_unopt, K:312-329: exact i32 block sum, then
 * sumf += (sum_i as f32 * d_w) * d_x, sequential in block order. */
float tnref_vec_dot_q4_0_q8_0(int64_t k, const uint8_t* w, const uint8_t* xq) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / QK; b++) {
        const uint8_t* wb = w + b * 18;
        const uint8_t* xb = xq + b * 34;
        int32_t sum_i = 0;
        for (int j = 0; j < QK / 2; j++) {
            int32_t v0 = (int32_t)(wb[2 + j] & 0x0f) - 8;
            int32_t v1 = (int32_t)(wb[2 + j] >> 4) - 8;
            sum_i += v0 * (int32_t)(int8_t)xb[2 + j] + v1 * (int32_t)(int8_t)xb[2 + j + QK / 2];
        }
        float dw = tnref_f16_to_f32((uint16_t)(wb[0] | (wb[1] << 8)));
        float dx = tnref_f16_to_f32((uint16_t)(xb[0] | (xb[1] << 8)));
        float t = (float)sum_i * dw;
        t = t * dx;
        sumf = sumf + t;
    }
    return sumf;
}

/* BlockQ8_0::vec_dot_unopt, K:738-757: exact i32 block sum of the two int8
 * code rows, then sumf += (sum_i as f32 * d_w) * d_x in block order. */
float tnref_vec_dot_q8_0_q8_0(int64_t k, const uint8_t* w, const uint8_t* xq) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / QK; b++) {
        const uint8_t* wb = w + b * 34;
        const uint8_t* xb = xq + b * 34;
        int32_t sum_i = 0;
        for (int j = 0; j < QK; j++) sum_i += (int32_t)(int8_t)wb[2 + j] * (int32_t)(int8_t)xb[2 + j];
        float dw = tnref_f16_to_f32((uint16_t)(wb[0] | (wb[1] << 8)));
        float dx = tnref_f16_to_f32((uint16_t)(xb[0] | (xb[1] << 8)));
        float t = (float)sum_i * dw;
        t = t * dx;
        sumf = sumf + t;
    }
    return sumf;
}

typedef float (*dot_fn)(int64_t, const uint8_t*, const uint8_t*);

typedef struct {
    int64_t m, k, n, c0, c1, wrow;
    const uint8_t* xq;
    const uint8_t* w;
    float* y;
    dot_fn dot;
} lin_job;

/* One worker's contiguous column range, ROW_TILE rows at a time: the loop
 * order of K:2512-2556. Every element is one vec_dot, so the order does not
 * change a bit of the result (tests/numerics/test_qgemm.py:64-87). */
static void* lin_worker(void* arg) {
    lin_job* j = (lin_job*)arg;
    const int64_t nb = j->k / QK;
    for (int64_t r0 = 0; r0 < j->m; r0 += 16) {
        int64_t r1 = r0 + 16 < j->m ? r0 + 16 : j->m;
        for (int64_t c = j->c0; c < j->c1; c++) {
            const uint8_t* wr = j->w + c * j->wrow;
            for (int64_t r = r0; r < r1; r++)
                j->y[r * j->n + c] = j->dot(j->k, wr, j->xq + r * nb * 34);
        }
    }
    return NULL;
}

/* Both weight formats quantise the activation rows to Q8_0 (their VecDotType,
 * K:281 and K:654) and differ only in the block dot and the weight's bytes
 * per block. */
static int q_linear(int64_t m, int64_t k, int64_t n, const float* x, const uint8_t* w, int64_t wblock,
                    dot_fn dot, const float* bias, float* y, int threads) {
    if (m < 0 || n < 0 || k <= 0 || k % QK) return -1;
    const int64_t nb = k / QK;
    uint8_t* xq = (uint8_t*)malloc((size_t)(m * nb * 34 + 1));
    if (!xq) return -1;
    for (int64_t r = 0; r < m; r++) tnref_q8_0_quantize(x + r * k, k, xq + r * nb * 34);
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    /* 4-column quads split evenly over the workers; the last worker also
     * takes the 1-3 tail columns (K:2557-2579 runs them on the caller). */
    int64_t quads = n / 4;
    int64_t per = (quads + threads - 1) / threads;
    pthread_t tid[256];
    int live[256];
    lin_job jobs[256];
    for (int t = 0; t < threads; t++) {
        int64_t c0 = t * per * 4, c1 = (t + 1) * per * 4;
        if (c0 > quads * 4) c0 = quads * 4;
        if (c1 > quads * 4) c1 = quads * 4;
        if (t == threads - 1) c1 = n;
        jobs[t] = (lin_job){m, k, n, c0, c1, nb * wblock, xq, w, y, dot};
        live[t] = threads > 1 && pthread_create(&tid[t], NULL, lin_worker, &jobs[t]) == 0;
        if (!live[t]) lin_worker(&jobs[t]);
    }
    for (int t = 0; t < threads; t++) if (live[t]) pthread_join(tid[t], NULL);
    free(xq);
    if (bias)
        for (int64_t r = 0; r < m; r++)
            for (int64_t c = 0; c < n; c++) y[r * n + c] = y[r * n + c] + bias[c];
    return 0;
}

int tnref_q4_0_linear(int64_t m, int64_t k, int64_t n, const float* x, const uint8_t* w,
                      const float* bias, float* y, int threads) {
    return q_linear(m, k, n, x, w, 18, tnref_vec_dot_q4_0_q8_0, bias, y, threads);
}

int tnref_q8_0_linear(int64_t m, int64_t k, int64_t n, const float* x, const uint8_t* w,
                      const float* bias, float* y, int threads) {
    return q_linear(m, k, n, x, w, 34, tnref_vec_dot_q8_0_q8_0, bias, y, threads);
}

void tnref_dense_linear(int64_t m, int64_t k, int64_t n, const float* x, const float* w, const float* bias,
                        float* y) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (int64_t t = 0; t < k; ++t) acc = fmaf(x[i * k + t], w[j * k + t], acc);
            y[i * n + j] = bias ? acc + bias[j] : acc;
        }
}

/* ------------------------------------------------------------------------ */
/* Q4_K weights with Q8_K activations                                        */
/* ------------------------------------------------------------------------ */
/* Layouts (K:153-190): Q4_K super-block of 256 = f16 d, f16 dmin, 12 bytes of
 * 6-bit scales and mins, 128 nibble bytes (144 bytes); Q8_K = f32 d, 256 int8
 * codes, 16 int16 sums of 16 codes (292 bytes). */
#define QKK 256

/* get_scale_min_k4, utils.rs:50-60. */
static void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* BlockQ4K::to_float, K:1722-1746: y = d*sc * nib - dmin*m per 32-element
 * sub-block; sub-blocks 2c and 2c+1 are the low and high nibbles of bytes
 * 32c..32c+31. */
void tnref_q4_k_dequantize(const uint8_t* blob, int64_t n, float* y) {
    for (int64_t b = 0; b < n / QKK; b++) {
        const uint8_t* in = blob + b * 144;
        const float d = tnref_f16_to_f32((uint16_t)(in[0] | (in[1] << 8)));
        const float dmin = tnref_f16_to_f32((uint16_t)(in[2] | (in[3] << 8)));
        const uint8_t* scales = in + 4;
        const uint8_t* qs = in + 16;
        float* out = y + b * QKK;
        for (int c = 0; c < 4; c++) {
            int sc, m;
            scale_min_k4(2 * c, scales, &sc, &m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            scale_min_k4(2 * c + 1, scales, &sc, &m);
            const float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; l++) out[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0x0f) - m1;
            for (int l = 0; l < 32; l++) out[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - m2;
        }
    }
}

/* BlockQ8K::from_float, K:2375-2413 (the non-NEON path): the first element of
 * the largest |x| sets iscale = -127/max; q = round-half-away(iscale*x)
 * clamped to [-128, 127] (NaN -> 0); d = 1/iscale in f32. */
void tnref_q8_k_quantize(const float* x, int64_t n, uint8_t* blob) {
    for (int64_t b = 0; b < n / QKK; b++) {
        const float* xs = x + b * QKK;
        uint8_t* out = blob + b * 292;
        float mx = 0.0f, amax = 0.0f;
        for (int j = 0; j < QKK; j++) {
            if (amax < fabsf(xs[j])) { amax = fabsf(xs[j]); mx = xs[j]; }
        }
        int8_t q[QKK];
        float d = 0.0f;
        if (amax == 0.0f) {
            memset(q, 0, sizeof q);
        } else {
            const float iscale = -127.0f / mx;
            for (int j = 0; j < QKK; j++) {
                float v = roundf(iscale * xs[j]);
                q[j] = (v != v) ? 0 : (v < -128.0f ? -128 : (v > 127.0f ? 127 : (int8_t)v));
            }
            d = 1.0f / iscale;
        }
        memcpy(out, &d, 4);
        memcpy(out + 4, q, QKK);
        for (int j = 0; j < QKK / 16; j++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += q[16 * j + i];
            int16_t s16 = (int16_t)(amax == 0.0f ? 0 : s);
            memcpy(out + 4 + QKK + 2 * j, &s16, 2);
        }
    }
}

/* BlockQ4K::vec_dot_unopt, K:1478-1558: per super-block, 8 exact i32 lane
 * sums aux32[l] = sum_j sc_j * sum_g q8[32j+8g+l] * nib[32j+8g+l], and
 * sumi = sum_j bsums[j] * m_{j/2}; then, in f32, sums[l] += (d_w*d_x) *
 * aux32[l] and sumf -= (dmin_w*d_x) * sumi; the result is
 * sumf + (((sums[0] + sums[1]) + ...) + sums[7]). */
float tnref_vec_dot_q4_k_q8_k(int64_t k, const uint8_t* w, const uint8_t* xq) {
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / QKK; b++) {
        const uint8_t* wb = w + b * 144;
        const uint8_t* xb = xq + b * 292;
        float yd;
        memcpy(&yd, xb, 4);
        const int8_t* q8 = (const int8_t*)(xb + 4);
        int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int32_t sumi = 0;
        for (int j = 0; j < 8; j++) {
            int sc, m;
            scale_min_k4(j, wb + 4, &sc, &m);
            for (int h = 0; h < 2; h++) {
                int16_t bs;
                memcpy(&bs, xb + 4 + QKK + 2 * (2 * j + h), 2);
                sumi += (int32_t)bs * m;
            }
            const uint8_t* qb = wb + 16 + 32 * (j / 2);
            for (int g = 0; g < 4; g++)
                for (int l = 0; l < 8; l++) {
                    const int e = 8 * g + l;
                    const int nib = (j & 1) ? (qb[e] >> 4) : (qb[e] & 0x0f);
                    aux32[l] += sc * (int32_t)(int16_t)(q8[32 * j + e] * nib);
                }
        }
        const float d = tnref_f16_to_f32((uint16_t)(wb[0] | (wb[1] << 8))) * yd;
        for (int l = 0; l < 8; l++) sums[l] = sums[l] + d * (float)aux32[l];
        const float dmin = tnref_f16_to_f32((uint16_t)(wb[2] | (wb[3] << 8))) * yd;
        sumf = sumf - dmin * (float)sumi;
    }
    float tot = 0.0f;
    for (int l = 0; l < 8; l++) tot = tot + sums[l];
    return sumf + tot;
}

/* llama.cpp's nearest_int (utils.rs:292-295): the 1.5*2^23 bit trick,
 * round to nearest, ties to even. */
static inline int nearest_int_even(float f) {
    const float v = f + 12582912.0f;
    return (int)(f32_bits(v) & 0x007fffff) - 0x00400000;
}

/* make_qkx2_quants, utils.rs:308-397, with rmin, rdelta, nstep, use_mad =
 * -1.0, 0.1, 20, false as BlockQ4K::from_float calls it. Every f32 operation
 * is separate and in the Rust order; `min` is overwritten by each better
 * candidate and used by the later steps; `l` keeps the best candidate's
 * levels. Returns the scale, *the_min = -min. */
static float make_qkx2(int nmax, const float* x, const float* w, uint8_t* l, float* the_min) {
    const int n = 32;
    const float rmin = -1.0f, rdelta = 0.1f;
    const int nstep = 20;
    float mn = x[0], mxv = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mxv) mxv = x[i];
        sum_w = sum_w + w[i];
        sum_x = sum_x + w[i] * x[i];
    }
    if (mn > 0.0f) mn = 0.0f;
    if (mxv == mn) {
        memset(l, 0, (size_t)n);
        *the_min = -mn;
        return 0.0f;
    }
    float iscale = (float)nmax / (mxv - mn);
    float scale = 1.0f / iscale;
    float best = 0.0f;
    for (int i = 0; i < n; i++) {
        int li = nearest_int_even(iscale * (x[i] - mn));
        li = li < 0 ? 0 : (li > nmax ? nmax : li);
        l[i] = (uint8_t)li;
        float diff = scale * (float)l[i] + mn - x[i];
        diff = diff * diff;
        best = best + w[i] * diff;
    }
    uint8_t laux[32];
    for (int is = 0; is <= nstep; is++) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (mxv - mn);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        for (int i = 0; i < n; i++) {
            int li = nearest_int_even(iscale * (x[i] - mn));
            li = li < 0 ? 0 : (li > nmax ? nmax : li);
            laux[i] = (uint8_t)li;
            const float lf = (float)li;
            sum_l = sum_l + w[i] * lf;
            sum_l2 = sum_l2 + w[i] * lf * lf;
            sum_xl = sum_xl + w[i] * lf * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0.0f) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0.0f) {
                this_min = 0.0f;
                this_scale = sum_xl / sum_l2;
            }
            float cur = 0.0f;
            for (int i = 0; i < n; i++) {
                float diff = this_scale * (float)laux[i] + this_min - x[i];
                diff = diff * diff;
                cur = cur + w[i] * diff;
            }
            if (cur < best) {
                memcpy(l, laux, (size_t)n);
                best = cur;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

/* BlockQ4K::from_float, K:1570-1654 (llama.cpp's quantize_row_q4_K_ref):
 * weights av_x + |x| with av_x = sqrt(sum(x^2)/32) per sub-block, the
 * make_qkx2 search per sub-block, 6-bit scales and mins as
 * min(63, (uint8_t)nearest_int(63/max * v)), then the final levels
 * nearest_int((x + dm)/d) clamped to [0, 15] for sub-blocks whose d is not
 * zero (the others keep the search's levels). */
void tnref_q4_k_quantize(const float* x, int64_t n, uint8_t* blob) {
    for (int64_t b = 0; b < n / QKK; b++) {
        const float* xs = x + b * QKK;
        uint8_t* out = blob + b * 144;
        uint8_t L[QKK];
        float scales[8], mins[8];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) {
            const float* xj = xs + 32 * j;
            float sum_x2 = 0.0f;
            for (int i = 0; i < 32; i++) sum_x2 = sum_x2 + xj[i] * xj[i];
            const float av_x = sqrtf(sum_x2 / 32.0f);
            float wts[32];
            for (int i = 0; i < 32; i++) wts[i] = av_x + fabsf(xj[i]);
            scales[j] = make_qkx2(15, xj, wts, L + 32 * j, &mins[j]);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        uint8_t sc[12];
        memset(sc, 0, sizeof sc);
        for (int j = 0; j < 8; j++) {
            uint8_t ls = (uint8_t)nearest_int_even(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)nearest_int_even(inv_min * mins[j]);
            if (ls > 63) ls = 63;
            if (lm > 63) lm = 63;
            if (j < 4) {
                sc[j] = ls;
                sc[j + 4] = lm;
            } else {
                sc[j + 4] = (uint8_t)((ls & 0x0f) | ((lm & 0x0f) << 4));
                sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
                sc[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        const uint16_t dh = tnref_f16_from_f32(max_scale / 63.0f);
        const uint16_t mh = tnref_f16_from_f32(max_min / 63.0f);
        for (int j = 0; j < 8; j++) {
            int s6, m6;
            scale_min_k4(j, sc, &s6, &m6);
            const float d = tnref_f16_to_f32(dh) * (float)s6;
            if (d == 0.0f) continue;
            const float dm = tnref_f16_to_f32(mh) * (float)m6;
            for (int i = 0; i < 32; i++) {
                int lv = nearest_int_even((xs[32 * j + i] + dm) / d);
                L[32 * j + i] = (uint8_t)(lv < 0 ? 0 : (lv > 15 ? 15 : lv));
            }
        }
        out[0] = (uint8_t)(dh & 0xff);
        out[1] = (uint8_t)(dh >> 8);
        out[2] = (uint8_t)(mh & 0xff);
        out[3] = (uint8_t)(mh >> 8);
        memcpy(out + 4, sc, 12);
        for (int c = 0; c < 4; c++)
            for (int i = 0; i < 32; i++)
                out[16 + 32 * c + i] = (uint8_t)(L[64 * c + i] | (L[64 * c + 32 + i] << 4));
    }
}

/* The Q4_K matmul: activation rows to Q8_K (its VecDotType, K:1445), then
 * the vec_dot above per output, the driver of K:2430-2582. */
typedef struct {
    int64_t m, k, n, c0, c1;
    const uint8_t* xq;
    const uint8_t* w;
    float* y;
} lin_k_job;

static void* lin_k_worker(void* arg) {
    lin_k_job* j = (lin_k_job*)arg;
    const int64_t nb = j->k / QKK;
    for (int64_t c = j->c0; c < j->c1; c++)
        for (int64_t r = 0; r < j->m; r++)
            j->y[r * j->n + c] = tnref_vec_dot_q4_k_q8_k(j->k, j->w + c * nb * 144, j->xq + r * nb * 292);
    return NULL;
}

int tnref_q4_k_linear(int64_t m, int64_t k, int64_t n, const float* x, const uint8_t* w, const float* bias,
                      float* y, int threads) {
    if (m < 0 || n < 0 || k <= 0 || k % QKK) return -1;
    const int64_t nb = k / QKK;
    uint8_t* xq = (uint8_t*)malloc((size_t)(m * nb * 292 + 1));
    if (!xq) return -1;
    for (int64_t r = 0; r < m; r++) tnref_q8_k_quantize(x + r * k, k, xq + r * nb * 292);
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    int64_t per = (n + threads - 1) / threads;
    pthread_t tid[256];
    int live[256];
    lin_k_job jobs[256];
    for (int t = 0; t < threads; t++) {
        int64_t c0 = t * per, c1 = (t + 1) * per;
        if (c0 > n) c0 = n;
        if (c1 > n) c1 = n;
        jobs[t] = (lin_k_job){m, k, n, c0, c1, xq, w, y};
        live[t] = threads > 1 && pthread_create(&tid[t], NULL, lin_k_worker, &jobs[t]) == 0;
        if (!live[t]) lin_k_worker(&jobs[t]);
    }
    for (int t = 0; t < threads; t++) if (live[t]) pthread_join(tid[t], NULL);
    free(xq);
    if (bias)
        for (int64_t r = 0; r < m; r++)
            for (int64_t c = 0; c < n; c++) y[r * n + c] = y[r * n + c] + bias[c];
    return 0;
}

/* ------------------------------------------------------------------------ */
/* SDPA default path                                                         */
/* ------------------------------------------------------------------------ */

/* One query row of A:10330-10423, written for a scalar type T:
 *   raw = q . k^T                      (candle matmul; summation order of the
 *                                       gemm crate is not restated: sequential)
 *   s   = raw * scale + 0 (+ -inf past the upper-left diagonal)   T:4886-4905
 *   s  += mask                          A:10383-10389
 *   m   = amax(s), NaN-propagating      T:4801
 *   w   = exp(s - m); sum = sum(w); p = w / sum; out = p . v
 *   lse = log(sum) + m                  A:10414-10420
 */
#define SDPA_BODY(T, EXP, LOG, NEGINF)                                                        \
    for (int64_t row = j->r0; row < j->r1; row++) {                                          \
        const int64_t i = row % L;                                                            \
        const int64_t bh = row / L;                                                           \
        const int64_t h = bh % Hq, b = bh / Hq;                                               \
        const int64_t kh = h / (Hq / Hkv);                                                    \
        const T* qr = q + row * D;                                                            \
        const T* kb = k + (b * Hkv + kh) * S * D;                                             \
        const T* vb = v + (b * Hkv + kh) * S * D;                                             \
        const T mul = (T)scale;                                                               \
        const int64_t keep = is_causal ? (i + 1 < S ? i + 1 : S) : S;                         \
        T mx = NEGINF;                                                                        \
        int nan_seen = 0;                                                                     \
        for (int64_t c = 0; c < S; c++) {                                                     \
            T raw = 0;                                                                        \
            for (int64_t d = 0; d < D; d++) raw = raw + qr[d] * kb[c * D + d];                \
            T s = raw * mul + (T)0;                                                           \
            if (c >= keep) s = s + NEGINF;                                                    \
            if (mask) s = s + mask[row * S + c];                                              \
            w[c] = s;                                                                         \
            if (s != s) nan_seen = 1;                                                         \
            else if (s > mx) mx = s;                                                          \
        }                                                                                     \
        if (nan_seen) mx = (T)NAN;                                                            \
        T sum = 0;                                                                            \
        for (int64_t c = 0; c < S; c++) { w[c] = EXP(w[c] - mx); sum = sum + w[c]; }          \
        for (int64_t c = 0; c < S; c++) w[c] = w[c] / sum;                                    \
        T* o = out + row * D;                                                                 \
        for (int64_t d = 0; d < D; d++) o[d] = 0;                                             \
        for (int64_t c = 0; c < S; c++) {                                                     \
            const T p = w[c];                                                                 \
            for (int64_t d = 0; d < D; d++) o[d] = o[d] + p * vb[c * D + d];                  \
        }                                                                                     \
        if (lse) lse[row] = LOG(sum) + mx;                                                    \
    }

typedef struct {
    int64_t B, Hq, Hkv, L, S, D, r0, r1;
    const void *q, *k, *v, *mask;
    int is_causal;
    double scale;
    void *out, *lse;
} sdpa_job;

static void* sdpa_worker_f32(void* arg) {
    sdpa_job* j = (sdpa_job*)arg;
    const int64_t Hq = j->Hq, Hkv = j->Hkv, L = j->L, S = j->S, D = j->D;
    const float *q = j->q, *k = j->k, *v = j->v, *mask = j->mask;
    float *out = j->out, *lse = j->lse;
    const int is_causal = j->is_causal;
    const double scale = j->scale;
    float* w = (float*)malloc((size_t)S * sizeof(float));
    if (!w) return NULL;
    SDPA_BODY(float, expf, logf, -INFINITY)
    free(w);
    return NULL;
}

static void* sdpa_worker_f64(void* arg) {
    sdpa_job* j = (sdpa_job*)arg;
    const int64_t Hq = j->Hq, Hkv = j->Hkv, L = j->L, S = j->S, D = j->D;
    const double *q = j->q, *k = j->k, *v = j->v, *mask = j->mask;
    double *out = j->out, *lse = j->lse;
    const int is_causal = j->is_causal;
    const double scale = j->scale;
    double* w = (double*)malloc((size_t)S * sizeof(double));
    if (!w) return NULL;
    SDPA_BODY(double, exp, log, -INFINITY)
    free(w);
    return NULL;
}

static int sdpa_run(void* (*fn)(void*), int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t S,
                    int64_t D, const void* q, const void* k, const void* v, const void* mask,
                    int is_causal, double scale, void* out, void* lse, int threads) {
    if (B < 0 || Hq < 0 || L < 0 || S <= 0 || D <= 0 || Hkv <= 0 || Hq % Hkv) return -1;
    int64_t rows = B * Hq * L;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (rows < threads) threads = rows > 0 ? (int)rows : 1;
    pthread_t tid[256];
    int live[256];
    sdpa_job jobs[256];
    int64_t per = (rows + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        int64_t r0 = t * per, r1 = (t + 1) * per;
        if (r0 > rows) r0 = rows;
        if (r1 > rows) r1 = rows;
        jobs[t] = (sdpa_job){B, Hq, Hkv, L, S, D, r0, r1, q, k, v, mask, is_causal, scale, out, lse};
        live[t] = threads > 1 && pthread_create(&tid[t], NULL, fn, &jobs[t]) == 0;
        if (!live[t]) fn(&jobs[t]);
    }
    for (int t = 0; t < threads; t++) if (live[t]) pthread_join(tid[t], NULL);
    return 0;
}

int tnref_sdpa_f32(int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t S, int64_t D,
                   const float* q, const float* k, const float* v, const float* mask,
                   int is_causal, double scale, float* out, float* lse, int threads) {
    return sdpa_run(sdpa_worker_f32, B, Hq, Hkv, L, S, D, q, k, v, mask, is_causal, scale, out,
                    lse, threads);
}

int tnref_sdpa_f64(int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t S, int64_t D,
                   const double* q, const double* k, const double* v, const double* mask,
                   int is_causal, double scale, double* out, double* lse, int threads) {
    return sdpa_run(sdpa_worker_f64, B, Hq, Hkv, L, S, D, q, k, v, mask, is_causal, scale, out,
                    lse, threads);
}
