/*
 * tnref -- CPU oracle for the q4_0 linear and the SDPA default path.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain C, the arithmetic
 * the reference (torchnative, Rust + vendored candle) performs on its CPU path,
 * so that the HIP library can be checked against it. It is linked or loaded
 * only by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, always as the checker and never as the thing measured or shipped.
 *
 * Every function names the reference file:line it follows. Paths are relative
 * to the reference checkout:
 *   K = torchnative/rust/vendor/candle-core/src/quantized/k_quants.rs
 *   A = torchnative/rust/torch_c/src/aten.rs
 *   T = torchnative/rust/torch_c/src/tensor.rs
 *   R = torchnative/rust/torch_c/src/reduced.rs
 */
#ifndef TNREF_H
#define TNREF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reduced floats (half 2.7.1 f16::from_f32 RNE; R:161-218 bf16 RNE, NaN quieted) ---- */
uint16_t tnref_f16_from_f32(float f);
float tnref_f16_to_f32(uint16_t h);
uint16_t tnref_bf16_from_f32(float f);
float tnref_bf16_to_f32(uint16_t h);
void tnref_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n);
void tnref_f32_to_bf16_n(const float* src, uint16_t* dst, int64_t n);
void tnref_bf16_to_f32_n(const uint16_t* src, float* dst, int64_t n);

/* ---- GGML block codecs (K:79-119 layouts, 18-byte Q4_0, 34-byte Q8_0) ---- */
void tnref_q4_0_quantize(const float* x, int64_t n, uint8_t* blob);   /* K:241-277 */
void tnref_q4_0_dequantize(const uint8_t* blob, int64_t n, float* y); /* K:219-239 */
void tnref_q8_0_quantize(const float* x, int64_t n, uint8_t* blob);   /* K:676-705 */
void tnref_q8_0_dequantize(const uint8_t* blob, int64_t n, float* y); /* K:659-674 */

/* ---- the quantised linear ---- */
/* One output element: K:312-329 (vec_dot_unopt, the x86_64 wheel's path). */
float tnref_vec_dot_q4_0_q8_0(int64_t k, const uint8_t* w_row, const uint8_t* xq_row);
/* K:2430-2582 driver + quant.rs:350-365 bias: y[m,n] = Q8_0(x) . W^T (+ bias).
 * threads <= 0 means one thread. Returns 0, or -1 on a bad shape. */
int tnref_q4_0_linear(int64_t m, int64_t k, int64_t n, const float* x, const uint8_t* w_blob,
                      const float* bias, float* y, int threads);
/* The dense control formats' linear (quant.rs:273-279: an f32/f16/bf16
 * "quantised" weight is widened up front and takes a plain matmul, candle
 * quantized/mod.rs:836-852). The reference's matmul order is the gemm crate's
 * and is not restated; this is the order the HIP library declares for
 * tn_dense_linear: y[m,n] = chain (+ bias[n]), chain = 0 then
 * fmaf(x[m,k], w[n,k], chain) for k = 0..K-1. w is f32 (already widened). */
void tnref_dense_linear(int64_t m, int64_t k, int64_t n, const float* x, const float* w, const float* bias,
                        float* y);
/* Q8_0 weights: K:738-757 (vec_dot_unopt) per output, the same driver. */
float tnref_vec_dot_q8_0_q8_0(int64_t k, const uint8_t* w_row, const uint8_t* xq_row);
int tnref_q8_0_linear(int64_t m, int64_t k, int64_t n, const float* x, const uint8_t* w_blob,
                      const float* bias, float* y, int threads);

/* ---- Q4_K weights (144-byte super-blocks of 256) with Q8_K activations (292 bytes) ---- */
void tnref_q4_k_quantize(const float* x, int64_t n, uint8_t* blob);   /* K:1570-1654 */
void tnref_q4_k_dequantize(const uint8_t* blob, int64_t n, float* y); /* K:1722-1746 */
void tnref_q8_k_quantize(const float* x, int64_t n, uint8_t* blob);   /* K:2375-2413 */
float tnref_vec_dot_q4_k_q8_k(int64_t k, const uint8_t* w_row, const uint8_t* xq_row); /* K:1478-1558 */
int tnref_q4_k_linear(int64_t m, int64_t k, int64_t n, const float* x, const uint8_t* w_blob,
                      const float* bias, float* y, int threads);

/* ---- SDPA, the default (flat) path: A:10330-10423 ----
 * q [B,Hq,L,D], k/v [B,Hkv,S,D] row-major; mask nullable, [B,Hq,L,S] row-major
 * in the accumulate type; out [B,Hq,L,D]; lse nullable [B,Hq,L]. GQA: query
 * head h reads key/value head h / (Hq/Hkv) (A:17106-17126). is_causal is
 * upper-left aligned (T:4886-4905). scale is used as given (callers pass
 * 1/sqrt(D) for the default, A:10216). */
int tnref_sdpa_f32(int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t S, int64_t D,
                   const float* q, const float* k, const float* v, const float* mask,
                   int is_causal, double scale, float* out, float* lse, int threads);
int tnref_sdpa_f64(int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t S, int64_t D,
                   const double* q, const double* k, const double* v, const double* mask,
                   int is_causal, double scale, double* out, double* lse, int threads);

#ifdef __cplusplus
}
#endif
#endif
