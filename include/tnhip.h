/*
 * tnhip -- MI355X (gfx950) HIP backend for torchnative's quantised-inference
 * hot path, exposed as a C ABI.
 *
 * The entry points are what a HIP device arm in torchnative's Rust dispatch
 * layer would bind over FFI (a `Repr::Hip` tensor arm and a `Where::Hip` arm in
 * `routed()`, beside the Vulkan arm). Each declaration names the reference
 * interface it replaces; reference paths are relative to the torchnative
 * checkout:
 *   quant.rs = torchnative/rust/torch_c/src/quant.rs
 *   aten.rs  = torchnative/rust/torch_c/src/aten.rs
 *   err.rs   = torchnative/rust/torch_c/src/err.rs
 *   device.rs, vulkan.rs, lib.rs in the same directory.
 *
 * Conventions
 *   - Every device pointer is owned by the caller. Outputs are caller-allocated.
 *     The library allocates only internal workspaces (grow-only, one per
 *     device and stream) for the activation quantisation of the prefill GEMM
 *     and the split-KV partials of decode attention.
 *   - `stream` is a hipStream_t (NULL = the default stream). Compute calls are
 *     asynchronous on it and never synchronise the host.
 *   - Every call returns a tn_status. On failure, tn_last_error() returns a
 *     thread-local message; TN_ENOTIMPL maps to Python's NotImplementedError
 *     (err.rs:11-13, a refusal by name), TN_EINVAL to RuntimeError with the
 *     reference's wording (err.rs:26-28), TN_EVALUE to ValueError. Nothing
 *     unsupported falls back to the host.
 *   - Tensors are dense row-major; the caller makes them contiguous first, as
 *     quant.rs:337-341 and aten.rs:10204 do.
 */
#ifndef TNHIP_H
#define TNHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int tn_status;
#define TN_OK 0
#define TN_EINVAL 1   /* RuntimeError, reference wording */
#define TN_ENOTIMPL 2 /* NotImplementedError: refused by name */
#define TN_EHIP 3     /* RuntimeError from the HIP runtime */
#define TN_EVALUE 4   /* ValueError (bad blob size, bad argument value) */

/* Element types (torch.float32, torch.bfloat16, torch.float16, torch.float64). */
#define TN_F32 0
#define TN_BF16 1
#define TN_F16 2
#define TN_F64 3

#define TN_ABI_VERSION 1

/* ---- errors, probe, counters (err.rs; device.rs:1671-1708 _cuda_counters /
 *      _cuda_probe; vulkan.rs:2138-2268 _vulkan_probe/_ops/_counters) ---- */
const char* tn_last_error(void);
int tn_abi_version(void);
/* Writes "name=...;arch=gfx950;cus=...;hbm_bytes=...;devices=N" for the
 * current device. Refuses with TN_ENOTIMPL, naming the reason (no driver, no
 * device, wrong arch), when the current device is not a gfx950. */
tn_status tn_probe(char* buf, size_t len);

typedef struct {
    uint64_t dispatches;     /* kernel launches */
    uint64_t bytes_uploaded; /* tn_memcpy_h2d */
    uint64_t host_downloads; /* tn_memcpy_d2h calls (host readbacks) */
    uint64_t bytes_downloaded;
    uint64_t refusals;       /* calls answered TN_ENOTIMPL */
    uint64_t workspace_bytes;
} tn_counters_t;
tn_status tn_counters(tn_counters_t* out);
tn_status tn_counters_reset(void);
/* Comma-separated op names this backend executes (the vulkan.rs:1100-1223
 * whitelist shape). Anything else is refused by name by the host arm. */
const char* tn_ops(void);

/* ---- device runtime (what a host with no other HIP user needs) ---- */
tn_status tn_device_count(int* n);
tn_status tn_set_device(int ordinal);
tn_status tn_get_device(int* ordinal);
tn_status tn_malloc(void** ptr, size_t bytes);
tn_status tn_free(void* ptr);
tn_status tn_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
tn_status tn_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
tn_status tn_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
tn_status tn_memset(void* dst, int value, size_t bytes, void* stream);
tn_status tn_stream_create(void** stream);
tn_status tn_stream_destroy(void* stream);
tn_status tn_stream_synchronize(void* stream);
tn_status tn_device_synchronize(void);
tn_status tn_event_create(void** event);
tn_status tn_event_destroy(void* event);
tn_status tn_event_record(void* event, void* stream);
tn_status tn_event_synchronize(void* event);
tn_status tn_event_elapsed_ms(float* ms, void* start, void* end);

/* ---- GGML q4_0 weights ----
 * A q4_0 weight [N, K] (K % 32 == 0, nb = K/32 blocks per row) lives on the
 * device as two planes, repacked from the 18-byte GGML blocks so that every
 * 16-byte nibble group is 16-byte aligned for 128-bit loads:
 *   qs: N * nb * 16 bytes, block (n, b) at byte (n*nb + b)*16, byte j holding
 *       element j in its low nibble and element j+16 in its high nibble;
 *   d : N * nb f16 scales (little-endian bit patterns), d[n*nb + b].
 * The GGML blob is always recoverable byte for byte (tn_q4_0_to_blob).
 * Replaces the device half of `_quantized_to` (quant.rs:384-405): blocks are
 * moved byte for byte and never re-quantised. */
tn_status tn_q4_0_from_blob(void* stream, const uint8_t* blob, int64_t n, int64_t k, uint8_t* qs,
                            uint16_t* d);
/* Inverse of tn_q4_0_from_blob, for `_quantized_blob` (quant.rs:213-221). */
tn_status tn_q4_0_to_blob(void* stream, const uint8_t* qs, const uint16_t* d, int64_t n,
                          int64_t k, uint8_t* blob);
/* `_quantize(t, "q4_0")` on the device: BlockQ4_0::from_float
 * (candle-core/src/quantized/k_quants.rs:241-277) on w f32 [n, k], bit-exact.
 * Refuses k % 32 != 0 by name (quant.rs:145-161). */
tn_status tn_q4_0_quantize(void* stream, const float* w, int64_t n, int64_t k, uint8_t* qs,
                           uint16_t* d);
/* `_dequantize` (quant.rs:180-189): BlockQ4_0::to_float (k_quants.rs:219-239),
 * bit-exact, out f32 [n, k]. */
tn_status tn_q4_0_dequantize(void* stream, const uint8_t* qs, const uint16_t* d, int64_t n,
                             int64_t k, float* out);
/* `_quantized_linear(input, weight, bias)` (quant.rs:286-369):
 *   y[m, n] = sum over blocks b, in block order, of
 *             ((float)(int dot of Q4_0 codes and Q8_0(x) codes) * d_w) * d_x
 *             (+ bias[n], added after the sum, quant.rs:350-365)
 * which is candle's k_quants::matmul (k_quants.rs:2430-2582) with the x86_64
 * wheel's vec_dot_unopt (k_quants.rs:312-329): each row of x is quantised to
 * Q8_0 (k_quants.rs:676-705) first. The result is bit-identical to that
 * arithmetic for every m (a batched call equals its one-row calls).
 *   x: [m, k] in x_dtype TN_F32 (the reference's only accepted activation) or
 *      TN_BF16 (widened exactly in-kernel); y: [m, n] in TN_F32 or TN_BF16
 *      (narrowed RNE); bias: nullable f32 [n].
 * Refuses other dtypes with TN_ENOTIMPL (quant.rs:299-306) and k % 32 != 0,
 * k <= 0 with TN_EINVAL "mat1 and mat2 shapes cannot be multiplied"
 * (quant.rs:322-332). */
tn_status tn_q4_0_linear(void* stream, const void* x, int x_dtype, int64_t m, int64_t k,
                         const uint8_t* qs, const uint16_t* d, int64_t n, const float* bias,
                         void* y, int y_dtype);

/* ---- scaled dot-product attention ----
 * `aten._scaled_dot_product_flash_attention_for_cpu(q, k, v, dropout_p=0.,
 * is_causal=False, *, attn_mask=None, scale=None) -> (out, logsumexp)`
 * (aten.rs:10092-10440), device half.
 *   q [B,Hq,L,D], k/v [B,Hkv,S,D] in `dtype` (TN_F32 or TN_BF16), dense.
 *   GQA: query head h reads key/value head h / (Hq/Hkv), indexed, not
 *   materialised (aten.rs:17106-17126); Hq % Hkv != 0 is refused by name.
 *   is_causal: upper-left aligned, row t attends keys 0..=t (aten.rs:10038-10041).
 *   attn_mask: nullable, [B,Hq,L,S] dense additive, in `mask_dtype` (the query
 *   dtype or TN_F32, aten.rs:10142-10148), added after scaling.
 *   scale: NaN selects 1/sqrt(D) (aten.rs:10216).
 *   out: [B,Hq,L,D] in `dtype` (row-major, aten.rs:10436-10437);
 *   lse: nullable f32 [B,Hq,L], logsumexp over the masked, scaled scores.
 * Accumulation is f32 for both dtypes (aten.rs:10196-10206); a bf16 run
 * narrows the probabilities to bf16 between the two products, as upstream's
 * blocked kernel does (flash.rs:503-516), and the output RNE.
 * Head dims 64 and 128 run; others are refused by name. */
tn_status tn_sdpa_fwd(void* stream, int dtype, const void* q, const void* k, const void* v,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t S, int64_t D,
                      const void* attn_mask, int mask_dtype, int is_causal, double scale,
                      void* out, float* lse);

/* Decode attention: one query token per sequence over a contiguous
 * per-sequence KV cache, the shape `PreallocatedLayer` keeps
 * (torchnative/python/torchnative/kernels/kv_cache.py:92-114): k/v cache
 * [B, Hkv, cap, D] with head stride cap*D, sequence b using keys 0..lens[b]-1.
 * Equals tn_sdpa_fwd with L = 1, non-causal, on the view k[:, :, :lens[b]]
 * (the reference passes attn_mask=None at L=1, sdpa_metal.rs:23-30).
 *   q [B, Hq, D], out [B, Hq, D] in `dtype`; lens: device int32 [B], each in
 *   [1, cap]; max_len: host upper bound of lens (sizes the split-KV grid);
 *   lse nullable f32 [B, Hq].
 * Split-KV with a combine pass; the partials live in the library workspace. */
tn_status tn_sdpa_decode(void* stream, int dtype, const void* q, const void* k_cache,
                         const void* v_cache, int64_t B, int64_t Hq, int64_t Hkv, int64_t cap,
                         int64_t D, const int32_t* lens, int64_t max_len, double scale,
                         void* out, float* lse);

#ifdef __cplusplus
}
#endif
#endif /* TNHIP_H */
