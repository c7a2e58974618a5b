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

/* Element types (torch.float32, torch.bfloat16, torch.float16, torch.float64,
 * and torch.bool for an attention mask: one byte, nonzero = true). */
#define TN_F32 0
#define TN_BF16 1
#define TN_F16 2
#define TN_F64 3
#define TN_BOOL 4

#define TN_ABI_VERSION 2

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
/* Graph capture of any sequence of calls on a created stream (the HIP-graph
 * counterpart of the reference's capture.rs:1-35): calls between begin and
 * end are recorded, not run; end returns an instantiated graph for
 * tn_graph_launch / tn_graph_destroy. A call that would allocate (a first
 * call of a shape, or one larger than any before it on this stream) is
 * refused while capturing; make it once before. Work buffers a graph
 * captured stay allocated until tn_stream_destroy. */
tn_status tn_stream_begin_capture(void* stream);
tn_status tn_stream_end_capture(void* stream, void** graph);
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

/* ---- GGML q8_0 weights ----
 * The other block format `_quantize` takes whose VecDotType is Q8_0
 * (k_quants.rs:652-757). Same two-plane layout as q4_0 with 32 code bytes
 * per block:
 *   qs: N * nb * 32 int8 codes, block (n, b) at byte (n*nb + b)*32, element j
 *       at byte j (the 34-byte GGML block minus its scale);
 *   d : N * nb f16 scales, d[n*nb + b].
 * Each function is its q4_0 namesake's counterpart, with the same refusals:
 *   from_blob / to_blob: the device half of `_quantized_to` / `_quantized_blob`
 *     (quant.rs:384-405, :213-221), byte for byte;
 *   quantize: BlockQ8_0::from_float (k_quants.rs:676-705) on w f32 [n, k];
 *   dequantize: BlockQ8_0::to_float (k_quants.rs:659-674);
 *   linear: `_quantized_linear` with BlockQ8_0::vec_dot_unopt
 *     (k_quants.rs:738-757): y[m, n] = sum over blocks, in block order, of
 *     ((float)(int dot of the two int8 code rows) * d_w) * d_x (+ bias[n]),
 *     bit-identical for every m. */
tn_status tn_q8_0_from_blob(void* stream, const uint8_t* blob, int64_t n, int64_t k, int8_t* qs,
                            uint16_t* d);
tn_status tn_q8_0_to_blob(void* stream, const int8_t* qs, const uint16_t* d, int64_t n,
                          int64_t k, uint8_t* blob);
tn_status tn_q8_0_quantize(void* stream, const float* w, int64_t n, int64_t k, int8_t* qs,
                           uint16_t* d);
tn_status tn_q8_0_dequantize(void* stream, const int8_t* qs, const uint16_t* d, int64_t n,
                             int64_t k, float* out);
tn_status tn_q8_0_linear(void* stream, const void* x, int x_dtype, int64_t m, int64_t k,
                         const int8_t* qs, const uint16_t* d, int64_t n, const float* bias,
                         void* y, int y_dtype);

/* ---- GGML q4_k weights ----
 * `_quantize(t, "q4_k")` and its matmul (k_quants.rs:1442-1746): 256-element
 * super-blocks of 144 bytes (f16 d, f16 dmin, 12 bytes of packed 6-bit scales
 * and mins, 128 nibble bytes), whose VecDotType is Q8_K (k_quants.rs:2336-2413).
 * On the device a q4_k weight [N, K] (K % 256 == 0) is ONE plane `w` of
 * N * K/256 super-blocks of 144 bytes, row-major. Each keeps its first 16
 * bytes; in each of its four 32-byte nibble chunks, GGML byte 8g + l
 * (g = 0..3, l = 0..7) is stored at byte 4l + g, so a dword holds the four
 * elements of one position mod 8 (the operands of one lane of the reference's
 * dot). Pointers must be 16-byte aligned.
 *   from_blob / to_blob: `_quantized_to` / `_quantized_blob` (quant.rs:384-405,
 *     :213-221): GGML bytes <-> the device layout, byte for byte;
 *   quantize: BlockQ4K::from_float (k_quants.rs:1570-1654; llama.cpp's
 *     quantize_row_q4_K_ref with make_qkx2_quants), bit-exact, x f32 [n, k];
 *   dequantize: BlockQ4K::to_float (k_quants.rs:1722-1746);
 *   linear: `_quantized_linear` with each row of x quantised to Q8_K
 *     (BlockQ8K::from_float, k_quants.rs:2375-2413) and every output
 *     BlockQ4K::vec_dot_unopt (k_quants.rs:1478-1558): eight f32 lane sums
 *     sums[l] += (d_w*d_x) * aux32[l] and sumf -= (dmin_w*d_x) * sumi, in
 *     super-block order, result sumf + (sums[0] + ... + sums[7]) summed in
 *     order (+ bias[n]); bit-identical for every m.
 * Refuses k % 256 != 0 with the reference's block-size message. */
tn_status tn_q4_k_from_blob(void* stream, const uint8_t* blob, int64_t n, int64_t k, uint8_t* w);
tn_status tn_q4_k_to_blob(void* stream, const uint8_t* w, int64_t n, int64_t k, uint8_t* blob);
tn_status tn_q4_k_quantize(void* stream, const float* x, int64_t n, int64_t k, uint8_t* w);
tn_status tn_q4_k_dequantize(void* stream, const uint8_t* w, int64_t n, int64_t k, float* out);
tn_status tn_q4_k_linear(void* stream, const void* x, int x_dtype, int64_t m, int64_t k,
                         const uint8_t* w, int64_t n, const float* bias, void* y, int y_dtype);

/* ---- dense formats f32 / f16 / bf16: the exactness control ----
 * `_quantize(t, "f32" | "f16" | "bf16")` stores the weight element by element
 * (candle k_quants.rs:2778-2910; block size 1) and `_quantized_linear` on such
 * a weight is a plain matmul on the weight widened to f32 (QMatMul::from_arc,
 * candle quantized/mod.rs:836-852), which must be bit-identical to the dense
 * linear (quant.rs:273-279). dtype / w_dtype is TN_F32, TN_F16 or TN_BF16;
 * anything else is refused with TN_ENOTIMPL.
 *   quantize: out[i] = x[i] (f32), half's round-to-nearest-even f16 / bf16
 *     narrowing (NaN keeps its high payload bits and is quieted);
 *   dequantize: half's exact widening to f32 (a NaN comes back quieted);
 *   linear: y[m, n] = chain(m, n) (+ bias[n], added once after the chain, as
 *     the addmm of nn.Linear's bias branch, aten.rs:9686-9700), where
 *     chain = 0, then fma(x[m, k], widen(w[n, k]), chain) for k = 0 .. K-1 in
 *     order: one fixed rounding sequence, equal for every m and every launch.
 *     x f32 [m, k], w [n, k] in w_dtype, bias nullable f32 [n], y f32 [m, n].
 *     The same function is the dense `F.linear` (bootstrap.py:13352-13357)
 *     with w_dtype TN_F32. */
tn_status tn_dense_quantize(void* stream, const float* x, int64_t count, int dtype, void* out);
tn_status tn_dense_dequantize(void* stream, const void* w, int dtype, int64_t count, float* out);
tn_status tn_dense_linear(void* stream, const float* x, int64_t m, int64_t k, const void* w, int w_dtype,
                          int64_t n, const float* bias, float* y);

/* ---- scaled dot-product attention ----
 * `aten._scaled_dot_product_flash_attention_for_cpu(q, k, v, dropout_p=0.,
 * is_causal=False, *, attn_mask=None, scale=None) -> (out, logsumexp)`
 * (aten.rs:10092-10440), device half.
 *   q [B,Hq,L,D], k/v [B,Hkv,S,D] in `dtype` (TN_F32, TN_BF16, TN_F16 or
 *   TN_F64), dense. An f64 query computes in f64 (plain kernel) and writes
 *   lse as f64 (`lse` then points at doubles); an f32 mask on it is refused
 *   by name (aten.rs:10160-10170).
 *   GQA: query head h reads key/value head h / (Hq/Hkv), indexed, not
 *   materialised (aten.rs:17106-17126); Hq % Hkv != 0 is refused by name.
 *   is_causal: upper-left aligned, row t attends keys 0..=t (aten.rs:10038-10041).
 *   attn_mask: nullable, additive, in `mask_dtype` (the query dtype or TN_F32,
 *   aten.rs:10142-10148; others are refused with the reference's wording),
 *   added after scaling (aten.rs:10383-10389). TN_BOOL takes a bool mask as
 *   F.sdpa's CIA body turns it into an additive one before this op,
 *   where(mask, 0, -inf) in the query's dtype (bootstrap.py:12918-12925,
 *   :13065-13066), read in place with no conversion pass. A row whose every
 *   key is masked gives NaN in out and lse, as the reference's row-max shift
 *   does (aten.rs:10392-10420).
 *   mask_strides: nullable host int64[4], the mask's element strides over
 *   (B, Hq, L, S); a zero stride broadcasts that dim, so a [L, S] or
 *   [B, 1, L, S] mask is read where it lies, as the reference broadcasts
 *   the mask onto the scores (aten.rs:10293-10303). NULL: dense [B,Hq,L,S].
 *   scale: NaN selects 1/sqrt(D) (aten.rs:10216).
 *   out: [B,Hq,L,D] in `dtype` (row-major, aten.rs:10436-10437);
 *   lse: nullable f32 [B,Hq,L], logsumexp over the masked, scaled scores.
 * Accumulation is f32 for every dtype (the reference widens bf16 and f16 to
 * f32, aten.rs:10196-10213); a bf16 or f16 run narrows the probabilities to
 * its dtype between the two products, as upstream's blocked kernel does
 * (flash.rs:503-516), and the output RNE.
 * Head dims 64 and 128 with scale >= 0 run on MFMA kernels; any other head
 * dim up to 256, or a negative scale, runs on a plain f32 kernel (f32
 * probabilities); a head dim past 256 is refused by name. */
tn_status tn_sdpa_fwd(void* stream, int dtype, const void* q, const void* k, const void* v,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t S, int64_t D,
                      const void* attn_mask, int mask_dtype, const int64_t* mask_strides,
                      int is_causal, double scale,
                      void* out, float* lse);

/* Decode attention: one query token per sequence over a contiguous
 * per-sequence KV cache, the shape `PreallocatedLayer` keeps
 * (torchnative/python/torchnative/kernels/kv_cache.py:92-114): k/v cache
 * [B, Hkv, cap, D] with head stride cap*D, sequence b using keys 0..lens[b]-1.
 * Equals tn_sdpa_fwd with L = 1, non-causal, on the view k[:, :, :lens[b]]
 * (the reference passes attn_mask=None at L=1, sdpa_metal.rs:23-30).
 *   q [B, Hq, D], out [B, Hq, D] and the caches in `dtype` (TN_BF16 or
 *   TN_F16, or TN_F32 for an f32 model); lens: device int32 [B], each in
 *   [1, cap];
 *   max_len: host upper bound of lens (sizes the split-KV grid);
 *   lse nullable f32 [B, Hq].
 * Head dims 64 and 128: split-KV with a combine pass, the partials in the
 * library workspace; any other head dim up to 256 runs on the plain kernel
 * (one workgroup per (sequence, head)). A sequence of length 0 gives NaN out
 * and -inf lse. */
tn_status tn_sdpa_decode(void* stream, int dtype, const void* q, const void* k_cache,
                         const void* v_cache, int64_t B, int64_t Hq, int64_t Hkv, int64_t cap,
                         int64_t D, const int32_t* lens, int64_t max_len, double scale,
                         void* out, float* lse);

/* tn_sdpa_decode for callers that cannot allocate device memory: code under
 * HIP graph capture, serving loops and harnesses that forbid hipMalloc. It
 * has no counterpart in the reference. Same arguments, same kernels and the
 * same result bit for bit as tn_sdpa_decode; its work buffer (split
 * partials and the stream-K prefix sums) is a fixed device array of
 * TN_DECODE_SCRATCH_BYTES per GPU, in the library's own device memory, held
 * until the process ends. It calls no hipMalloc or hipFree. A call whose
 * work buffer would exceed the array refuses with TN_EVALUE naming both
 * sizes (e.g. config 4's B=16, 32/8 heads, head dim 128 needs about 4.5 MB).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (on different streams) race, so serialise them. */
#define TN_DECODE_SCRATCH_BYTES (8u << 20)
tn_status tn_sdpa_decode_noalloc(void* stream, int dtype, const void* q, const void* k_cache,
                                 const void* v_cache, int64_t B, int64_t Hq, int64_t Hkv, int64_t cap,
                                 int64_t D, const int32_t* lens, int64_t max_len, double scale,
                                 void* out, float* lse);

/* ---- decode-step ops ----
 * The per-token aten ops around the linear and the attention in a Llama-style
 * decoder step, f32, as the reference runs them for an f32 model
 * (`transformers`' LlamaForCausalLM over torch._C; the op census of a decode
 * step in profile_llama_cpp.json). All tensors are dense row-major device
 * memory; positions and token ids are device int32, so a sequence of steps
 * can be captured as a graph once and replayed. */

/* `aten.embedding.default` (aten.rs:11980-12040): out[i, :] = table[ids[i], :]
 * for an f32 table [vocab, dim] and device int32 ids [m]. An id outside
 * [0, vocab) gives a row of NaN (a device id cannot be checked on the host
 * without a synchronisation). */
tn_status tn_embedding(void* stream, const int32_t* ids, int64_t m, const float* table, int64_t vocab,
                       int64_t dim, float* out);

/* LlamaRMSNorm in f32 through the reference's ops: pow(x, 2) (aten.rs:4656),
 * mean over the row = sum then divide (aten.rs:15812), + eps, rsqrt = sqrt
 * then reciprocal (aten.rs:11112-11133), x * r, then weight * that.
 * x, y [m, n]; weight [n]; y may alias x. The row sum is a tree, not the
 * reference's order: equal within the f32 tolerance, not bitwise. */
tn_status tn_rmsnorm(void* stream, const float* x, int64_t m, int64_t n, const float* weight, double eps,
                     float* y);

/* Rotary embedding in place (LlamaRotaryEmbedding + apply_rotary_pos_emb:
 * x * cos + rotate_half(x) * sin, cos/sin of pos * inv_freq in f32, the
 * angle table duplicated over the two halves). x [m, heads, d]; token t is
 * at position pos[t] (device int32 [m]); inv_freq f32 [d/2]
 * (1 / theta^(2i/d), computed by the caller as the model does). */
tn_status tn_rope(void* stream, float* x, int64_t m, int64_t heads, int64_t d, const float* inv_freq,
                  const int32_t* pos);

/* silu(gate) * up: candle's silu x / (1 + exp(-x)) (candle-core op.rs:782-784,
 * aten.rs:15360-15384), then aten.mul.Tensor. out may alias gate or up. */
tn_status tn_silu_mul(void* stream, const float* gate, const float* up, int64_t n, float* out);

/* `aten.add.Tensor` on f32 vectors: out = a + b; out may alias a or b. */
tn_status tn_add(void* stream, const float* a, const float* b, int64_t n, float* out);

/* `aten.argmax.default` over the last dim of x [m, n] f32 (aten.rs:11927-11975
 * with first_extremum_index, aten.rs:16705-16741): the first maximal index,
 * or the first NaN's if the row holds one. out: device int32 [m]. */
tn_status tn_argmax(void* stream, const float* x, int64_t m, int64_t n, int32_t* out);

/* KV-cache append (PreallocatedLayer.update, kernels/kv_cache.py:92-114):
 * rows k, v [m, hkv, d] f32 go to k_cache, v_cache [hkv, cap, d] at positions
 * pos0[0] + i. Positions at or past cap are not written (the caller sizes
 * the cache). */
tn_status tn_kv_append(void* stream, const float* k, const float* v, int64_t m, int64_t hkv, int64_t d,
                       float* k_cache, float* v_cache, int64_t cap, const int32_t* pos0);

/* One f32 activation row through a q4_0 linear with the decode step's
 * neighbouring ops fused in, bit-identical to running them separately:
 *   prologue TN_PRO_NONE     x [k]
 *            TN_PRO_RMSNORM  x [k] -> tn_rmsnorm(x, prologue_w [k], eps)
 *            TN_PRO_SILU     x [2k] = gate | up -> tn_silu_mul(gate, up)
 *   then y [n] = tn_q4_0_linear of that row (no bias),
 *   then, if resid is non-null, y = tn_add(resid [n], y).
 * TN_PRO_RMSNORM_SILU is the MLP's first half instead: x [k] ->
 * tn_rmsnorm(x, prologue_w, eps); the weight holds [gate; up], 2n rows; the
 * 2n outputs g | u of tn_q4_0_linear give y [n] = tn_silu_mul(g, u) (resid
 * must be null), so the down projection's input leaves the GEMV finished.
 * The reference runs these as separate ops (LlamaRMSNorm, the SiLU-gated
 * MLP and the residual adds of modeling_llama.py around
 * `_quantized_linear`, quant.rs:286-369); the fusion saves the launches and
 * the round trips of the intermediate rows. y may alias resid (the decoder's
 * in-place residual), never x. k must be a multiple of 32, at most 24576. */
#define TN_PRO_NONE 0
#define TN_PRO_RMSNORM 1
#define TN_PRO_SILU 2
#define TN_PRO_RMSNORM_SILU 3
tn_status tn_q4_0_linear_decode(void* stream, const float* x, int64_t k, int prologue, const float* prologue_w,
                                double eps, const uint8_t* qs, const uint16_t* d, int64_t n, const float* resid,
                                float* y);

/* ---- greedy decode of a q4_0 Llama-style decoder ----
 * No single reference function: the reference runs this step as
 * transformers' LlamaForCausalLM.forward over its torch._C ops, with every
 * nn.Linear swapped for QuantizedLinear (quant/__init__.py:100-365), then
 * the greedy argmax of generate(). tn_llama_step launches one whole step of
 * that on the device -- five launches per layer: tn_q4_0_linear_decode with
 * the norms, SiLU and residual adds fused in, one RoPE + KV-append kernel,
 * and the f32 decode attention -- so that a caller (or a captured graph)
 * pays one call per token:
 *   h = embed[token]; per layer: x = rmsnorm(h, ln1); qkv = x W_qkv^T;
 *   rope(q, k at pos); append k, v; a = attention(q, cache[0..pos]);
 *   h += a W_o^T; x = rmsnorm(h, ln2); gu = x W_gate_up^T;
 *   h += (silu(gate) * up) W_down^T (the SiLU in the gate_up launch, as
 *   TN_PRO_RMSNORM_SILU); then logits = rmsnorm(h, norm) W_lm^T,
 *   next = argmax(logits).
 * The projections are stacked row-wise (q|k|v and gate|up): each output
 * row of the q4 linear is computed on its own, so stacking changes no bit.
 * Step state lives on the device in `state` (int32 [4]): [0] the position
 * of the token being processed, [1] = [0] + 1 (the KV length), [2] that
 * token's id, [3] the argmax of the step. After the step [0] and [1]
 * advance by one and [2] becomes the next input: prompt[[0]] while the
 * prompt lasts, else the argmax; it is also stored in tokens[[0]] (the
 * caller writes tokens[0]). */
typedef struct tn_q4_weight {
    const uint8_t* qs; /* [n][k/32][16] nibble bytes */
    const uint16_t* d; /* [n][k/32] f16 scales */
} tn_q4_weight;

typedef struct tn_llama_layer {
    tn_q4_weight qkv;     /* [(n_heads + 2 n_kv_heads) head_dim, hidden] */
    tn_q4_weight o;       /* [hidden, n_heads head_dim] */
    tn_q4_weight gate_up; /* [2 inter, hidden]: gate rows, then up rows */
    tn_q4_weight down;    /* [hidden, inter] */
    const float* ln1;     /* input_layernorm weight [hidden] */
    const float* ln2;     /* post_attention_layernorm weight [hidden] */
    float* k_cache;       /* [n_kv_heads, cap, head_dim] f32 */
    float* v_cache;
} tn_llama_layer;

typedef struct tn_llama {
    int64_t n_layers, hidden, n_heads, n_kv_heads, head_dim, inter, vocab;
    int64_t cap;        /* KV capacity = the longest sequence (prompt + generated) */
    double eps;         /* RMSNorm epsilon */
    const float* embed; /* [vocab, hidden] */
    const float* norm;  /* final norm weight [hidden] */
    tn_q4_weight lm_head;   /* [vocab, hidden] */
    const float* inv_freq;  /* [head_dim / 2] */
    const tn_llama_layer* layers; /* host array [n_layers] */
    const int32_t* prompt;  /* device [prompt_len] */
    int64_t prompt_len;
    int32_t* state;     /* device [4], see above */
    int32_t* tokens;    /* device [cap]: tokens[p] = the input token at position p */
    float* logits;      /* device [vocab], the last step's logits */
    float* work;        /* device scratch, tn_llama_work_floats() floats */
} tn_llama;

/* Floats of device scratch tn_llama_step needs for this model. */
int64_t tn_llama_work_floats(const tn_llama* model);
/* One decode step of `model` on `stream` (see above). Allocates nothing. */
tn_status tn_llama_step(void* stream, const tn_llama* model);
/* Captures `steps` consecutive calls of tn_llama_step into a HIP graph
 * (hipGraphExec_t returned in *graph) for replay with tn_graph_launch. The
 * model's buffers must stay valid while the graph lives. */
tn_status tn_llama_capture(void* stream, const tn_llama* model, int64_t steps, void** graph);
tn_status tn_graph_launch(void* stream, void* graph);
tn_status tn_graph_destroy(void* graph);

/* The prompt in one batched pass (the reference's prefill: one
 * LlamaForCausalLM.forward over the prompt, timed on its own in
 * tests/bench/bench_llama_cpp.py:484-523): the model's first `tokens`
 * prompt tokens run through every layer at once -- RMSNorm rows, the q4_0
 * linears as GEMMs (M = tokens), RoPE, the K/V rows into the caches at
 * positions 0 .. tokens-1, the causal f32 SDPA prefill, the SiLU-gated MLP
 * and the residual adds -- then the last position's logits, their argmax
 * and the state's advance exactly as tn_llama_step ends, so tn_llama_step
 * continues at position `tokens`. 1 <= tokens <= prompt_len <= cap. `work`
 * holds tn_llama_prefill_work_floats(model, tokens) floats; the model's
 * own work buffer is used too. The q4 GEMM allocates its stream workspace
 * on a first call (not capturable then). */
int64_t tn_llama_prefill_work_floats(const tn_llama* model, int64_t tokens);
tn_status tn_llama_prefill(void* stream, const tn_llama* model, int64_t tokens, float* work);

#ifdef __cplusplus
}
#endif
#endif /* TNHIP_H */
