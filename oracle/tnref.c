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
